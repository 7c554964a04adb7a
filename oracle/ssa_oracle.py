"""CPU oracle for SSA's routed block-sparse attention -- TEST INFRASTRUCTURE ONLY.

A NumPy restatement of the reference algorithm, used as the checker by tests/, by
__graft_entry__.smoke() and as the CPU baseline leg of bench.py. Nothing in the product path
(ssa_amd/) imports it, and it is never a fallback for the HIP kernels.

Numerics. Block statistics, query-block means and the router's inner products are accumulated
in float64 from the float32 operands and rounded once to float32, with elementwise products
(q*q, q*q*q) and the final combination r = E1 + c2*E2 (+ c3*E3) rounded to float32 exactly where
the reference's float32 torch code rounds. These are the correctly rounded values of the
reference formula; the reference's own float32 reductions differ from them by a few ulps, which
can only change a selection where two candidate scores are within that noise (see
`selection_gap`). Attention is exact masked softmax in float64.

Pinning (what checks each function; details in tests/test_oracle.py):
  block_stats / qmean    closed form on hand-built blocks; pad exclusion; golden fixtures via
                         the selections they induce.
  scores / select_rows   reference golden fixtures (tests/golden/, produced by the reference
                         itself in float32) -- equal except on rows `selection_gap` flags as
                         within float32 noise; brute-force enumeration on tiny rows; budget=1 ->
                         all causal blocks; beta=0 -> centroid routing.
  sparse_attention       reference golden outputs (FlexAttention / analytic path); full budget
                         == dense causal softmax; needle known-answer test.
  decode_attend          equals the prefill row for the same blocks; golden analytic q_len=1 rows.
  masked_route /         reference ssa_masked fixtures (float32 forward and autograd gradients);
  masked_forward /       planted slips (biased variance, pad rows dropped, complete-block
  masked_grads           candidates) fail them; full selection == dense causal and torch autograd;
                         central differences on a sparse GQA case.
  ivf_build / ivf_search  (faiss, the reference's IVF dependency, is absent: no fixtures.) Every
  / ivf_route            list probed and search_k = nb reduces the search to brute-force top_c
                         of <q̄_i, μ_j> over j <= i; a hand-built case where the search_k cut
                         holds only future blocks (filtering before the cut would select past
                         ones); full budget -> all causal blocks; planted well-separated
                         clusters are recovered exactly; the final lists partition the blocks,
                         ascending, each member at its argmax centroid; Jaccard >= 0.6 against
                         the flat router on the clustered geometry of the reference's own test.
  tree_build /           (the reference has no tests or fixtures for ssa/treecode.py.) The
  tree_descend           admissible invariant of its own validation (treecode.py:141-157: every
                         node's bound >= the largest key score below it) on random and clustered
                         keys; brute-force leaf statistics; a beam wide enough to hold every node
                         reduces the descent to the flat top_c of the leaf bounds; recall climbs
                         with W to the flat ceiling (treecode.py:160-200); the causal mask keeps
                         every selected leaf at or before q_pos.
  CascadeOracle /        (faiss is absent and the reference holds no fixtures for
  ccc_* (cascade)        ssa/cascade_router.py; tests/test_oracle_ccc.py.) Its own mechanics and
                         soundness tests restated: exhaustive search equals the brute-force
                         sub-block max-pool (float64); one chunk or 2-block chunks select alike;
                         causal / own-block / unique lists; every certified row holds the exact
                         top-k routing blocks with a built index (clustered and random keys),
                         and dropping the radii from the bound breaks that; incremental radii
                         bound every member and are exact after a rebuild; escalation never
                         lowers the certified rate and raises it on random keys; the outlier
                         channel catches a hidden 12 u key the sub-block routing misses; a
                         starved probe fails closed. Closed forms: group means, outlier order,
                         Lloyd update of two separated clusters.
"""
from __future__ import annotations

import math

import numpy as np

# ---------------------------------------------------------------------------------------------
# a1 / a2: block summaries
# ---------------------------------------------------------------------------------------------


def block_stats(x: np.ndarray, block: int, mode: str = "pop", n_real: int | None = None):
    """x (B, H, n, d) -> mu, var, m3 (B, H, nb, d) float32, nb = ceil(n/block).

    mode "pop": rows < n_real counted, cnt = max(1, #counted), var and m3 divide by cnt
      -- ssa/ssa_kernel.py:80-91 (block_route_budget), ssa/gemma_ssa.py:65-82 (_block_stats).
    mode "unbiased": var divides by cnt - 1 -- ssa/ssa_kernel.py:43,47 (kb.var(3)).
    """
    B, H, n, d = x.shape
    nb = -(-n // block)
    nr = n if n_real is None else min(n, int(n_real))
    outs = [np.empty((B, H, nb, d), dtype=np.float32) for _ in range(3)]
    # blocks are independent: taken in chunks of whole blocks to bound the float64 temporaries
    step = max(1, (1 << 22) // max(1, B * H * block * d))
    for c0 in range(0, nb, step):
        c1 = min(nb, c0 + step)
        r0, r1 = c0 * block, min(n, c1 * block)
        xp = np.zeros((B, H, (c1 - c0) * block, d), dtype=np.float64)
        xp[:, :, :r1 - r0] = x[:, :, r0:r1]
        valid = np.zeros(((c1 - c0) * block,), dtype=bool)
        valid[:max(0, min(nr, r1) - r0)] = True
        xb = xp.reshape(B, H, c1 - c0, block, d)
        vb = valid.reshape(c1 - c0, block)[None, None, :, :, None]
        cnt_rows = vb.sum(3)                                      # (1,1,nb,1)
        cnt = np.maximum(cnt_rows, 1).astype(np.float64)
        s1 = np.where(vb, xb, 0.0).sum(3)
        mean = s1 / cnt
        cen = np.where(vb, xb - mean[:, :, :, None, :], 0.0)
        s2 = (cen * cen).sum(3)
        s3 = (cen * cen * cen).sum(3)
        vden = cnt - 1.0 if mode == "unbiased" else cnt
        with np.errstate(divide="ignore", invalid="ignore"):
            var = s2 / vden
        outs[0][:, :, c0:c1] = mean
        outs[1][:, :, c0:c1] = var
        outs[2][:, :, c0:c1] = s3 / cnt
    return outs[0], outs[1], outs[2]


def qmean(q: np.ndarray, block: int) -> np.ndarray:
    """Query-block summary q.view(B,H,nb,block,d).float().mean(3), pad rows counted as zeros
    (ssa/ssa_kernel.py:44,79; the caller pads with zeros at ssa/gemma_ssa.py:149)."""
    B, H, n, d = q.shape
    nb = -(-n // block)
    out = np.empty((B, H, nb, d), dtype=np.float32)
    step = max(1, (1 << 22) // max(1, B * H * block * d))  # whole blocks per chunk
    for c0 in range(0, nb, step):
        c1 = min(nb, c0 + step)
        r0, r1 = c0 * block, min(n, c1 * block)
        qp = np.zeros((B, H, (c1 - c0) * block, d), dtype=np.float64)
        qp[:, :, :r1 - r0] = q[:, :, r0:r1]
        out[:, :, c0:c1] = qp.reshape(B, H, c1 - c0, block, d).sum(3) / block
    return out


# ---------------------------------------------------------------------------------------------
# a3: cumulant score
# ---------------------------------------------------------------------------------------------


def scores(rows: np.ndarray, mu: np.ndarray, var: np.ndarray | None, coef2: float,
           m3: np.ndarray | None = None, coef3: float = 0.0) -> np.ndarray:
    """r[b,h,i,c] = fl32(fl32(<q,mu_c>) + fl32(c2 * fl32(<q*q, var_c>))) [+ fl32(c3*fl32(<q^3,m3_c>))]
    for rows (B, Hq, R, d) and summaries (B, Hkv, nbk, d); query head h uses key head
    h // (Hq/Hkv). Reference: ssa/ssa_kernel.py:96-99 (block_route_budget), :45-47 (block_route),
    ssa/gemma_ssa.py:99-102 (_selection_mask)."""
    B, Hq, R, d = rows.shape
    Hkv = mu.shape[1]
    G = Hq // Hkv
    q = rows.astype(np.float32)
    q2 = (q * q).astype(np.float32)                    # elementwise fp32 products, as torch
    out = np.empty((B, Hq, R, mu.shape[2]), dtype=np.float32)
    c2 = np.float32(coef2)
    c3 = np.float32(coef3)
    for b in range(B):
        for h in range(Hq):
            kh = h // G
            e1 = (q[b, h].astype(np.float64) @ mu[b, kh].astype(np.float64).T).astype(np.float32)
            r = e1
            if var is not None and coef2 != 0.0:
                e2 = (q2[b, h].astype(np.float64) @ var[b, kh].astype(np.float64).T).astype(np.float32)
                r = (e1 + (c2 * e2).astype(np.float32)).astype(np.float32)
            if m3 is not None:
                q3 = (q2[b, h] * q[b, h]).astype(np.float32)
                e3 = (q3.astype(np.float64) @ m3[b, kh].astype(np.float64).T).astype(np.float32)
                r = (r + (c3 * e3).astype(np.float32)).astype(np.float32)
            out[b, h] = r
    return out


def score_keys(r: np.ndarray) -> np.ndarray:
    """Order-preserving uint32 keys of fp32 scores: -0 folded onto +0 (torch.topk treats them as
    equal), NaN above +inf (torch.topk's NaN-is-largest)."""
    r = np.where(r == 0.0, np.float32(0.0), r).astype(np.float32)
    u = r.view(np.uint32)
    k = np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)
    return np.where(np.isnan(r), np.uint32(0xFFFFFFFF), k).astype(np.uint32)


# ---------------------------------------------------------------------------------------------
# a4 / a5: selection and compaction
# ---------------------------------------------------------------------------------------------


def _keep_budget(frac: float, nvis: int) -> int:
    """max(1, ceil(fl32(frac) * fl32(nvis))) computed in float32 (ssa/ssa_kernel.py:105-106,
    ssa/gemma_ssa.py:117-118)."""
    return max(1, int(math.ceil(float(np.float32(frac) * np.float32(nvis)))))


def row_geometry(mode: str, i: int, nbk: int, top_c, budget_frac, query_pos=0, block=1):
    """(cmax, keep, own) of row i: candidates are blocks [0, cmax), `keep` of them are kept (ties
    to the lowest index), and the own block with its `local` predecessors is always added.
    budget: c < i (ssa/ssa_kernel.py:101-106); flat: c <= i (ssa/ssa_kernel.py:48-52);
    query: blocks complete at pos = query_pos + i (ssa/gemma_ssa.py:104-118); started: blocks
    begun at pos, its own included (ssa/ssa_swap.py:44-45)."""
    if mode == "budget":
        cmax, own = min(i, nbk), i
    elif mode == "flat":
        cmax, own = min(i + 1, nbk), i
    elif mode == "query":
        pos = query_pos + i
        cmax, own = min((pos + 1) // block, nbk), pos // block
    elif mode == "started":  # ssa/ssa_swap.py:44-45: block j visible once it has begun
        pos = query_pos + i
        cmax, own = min(pos // block + 1, nbk), pos // block
    else:
        raise ValueError(mode)
    if mode == "flat" or top_c is not None:
        keep = int(top_c)
    else:
        keep = _keep_budget(budget_frac, cmax)
    return cmax, keep, own


def select_rows(r: np.ndarray, mode: str, top_c, budget_frac: float, local: int,
                query_pos: int = 0, block: int = 1):
    """r (B, Hq, R, nbk) fp32 scores -> list-of-lists of selected block ids per row (ascending):
    top-min(keep, cmax) candidates by (score desc, index asc) | own-local..own, clipped to
    [0, min(own, nbk-1)]. Reference: ssa/ssa_kernel.py:101-116, :48-55; ssa/gemma_ssa.py:119-131."""
    B, Hq, R, nbk = r.shape
    keys = score_keys(r)
    out = np.empty((B, Hq, R), dtype=object)
    for i in range(R):
        for b in range(B):
            for h in range(Hq):
                out[b, h, i] = select_row(keys[b, h, i], i, mode, top_c, budget_frac, local,
                                          query_pos, block)
    return out


def select_row(keys: np.ndarray, i: int, mode: str, top_c, budget_frac: float, local: int,
               query_pos: int = 0, block: int = 1) -> list:
    """Selection of the single row i from its score keys (nbk,) (score_keys of the fp32 scores),
    with the geometry of row_geometry; the per-row body of select_rows."""
    nbk = keys.shape[0]
    cmax, keep, own = row_geometry(mode, i, nbk, top_c, budget_frac, query_pos, block)
    k = min(keep, cmax)
    lo, hi = max(0, own - local), min(own, nbk - 1)
    if k >= cmax:
        pick = set(range(cmax))
    elif k > 0:
        order = np.argsort(-keys[:cmax].astype(np.int64), kind="stable")
        pick = set(order[:k].tolist())
    else:
        pick = set()
    return sorted(pick | set(range(lo, hi + 1)))


def compact(sel_lists, W: int | None = None):
    """List-of-lists -> (kv_num (B,Hq,R) int32, kv_idx (B,Hq,R,W) int32, ascending, pad 0)."""
    B, Hq, R = sel_lists.shape
    if W is None:
        W = max(1, max(len(x) for x in sel_lists.ravel()))
    kv_num = np.zeros((B, Hq, R), dtype=np.int32)
    kv_idx = np.zeros((B, Hq, R, W), dtype=np.int32)
    for idx in np.ndindex(B, Hq, R):
        ids = sel_lists[idx]
        kv_num[idx] = len(ids)
        kv_idx[idx][:len(ids)] = ids
    return kv_num, kv_idx


def project(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """fl32(x @ w) with the products summed in float64 (x (..., din), w (din, dout)): the
    projections qb @ W_q and mu @ W_k of ssa/ssa_kernel.py:92-94, rounded once."""
    return (x.astype(np.float64) @ np.asarray(w, dtype=np.float64)).astype(np.float32)


def pool_max(r: np.ndarray, pool: int) -> np.ndarray:
    """Max over each run of `pool` consecutive sub-block scores (last axis): the max-pool
    rs.view(..., nb, spb).amax(-1) of ssa/ssa_kernel.py:100 (NaN propagates like torch.amax)."""
    if pool == 1:
        return r
    return r.reshape(*r.shape[:-1], r.shape[-1] // pool, pool).max(-1)


def route_budget(q, k, block, budget_frac=0.25, top_c=None, local=1, beta=2.0, edgeworth=False,
                 n_real=None, sub=None, proj=None):
    """block_route_budget (ssa/ssa_kernel.py:61-119) -> (kv_num, kv_idx compact). q (B,Hq,n,d),
    k (B,Hkv,n,d), query head h reads key head h // (Hq/Hkv). `sub`: key summaries over
    sub-blocks of that size, scores max-pooled to the block (:74-78,100). `proj`: a (d, d')
    matrix or a pair (W_q, W_k); the score is then <qb W_q, mu W_k> only (:92-94)."""
    qb = qmean(q, block)
    sub_sz = block if sub is None else int(sub)
    mu, var, m3 = block_stats(k, sub_sz, "pop", n_real)
    if proj is not None:
        wq, wk = proj if isinstance(proj, tuple) else (proj, proj)
        r = scores(project(qb, wq), project(mu, wk), None, 0.0)
    else:
        r = scores(qb, mu, var, 0.5 * beta, m3 if edgeworth else None, beta ** 2 / 6.0)
    r = pool_max(r, block // sub_sz)
    return compact(select_rows(r, "budget", top_c, budget_frac, local))


def route_flat(q, k, block, top_c=8, local=1, routing="cumulant"):
    """block_route (ssa/ssa_kernel.py:37-58) -> (kv_num, kv_idx compact)."""
    qb = qmean(q, block)
    mu, var, _ = block_stats(k, block, "unbiased")
    cum = routing == "cumulant"
    r = scores(qb, mu, var if cum else None, 0.5 if cum else 0.0)
    return compact(select_rows(r, "flat", top_c, 0.0, local))


def route_query(qrows, k, block, pos0, top_c=None, budget_frac=0.25, local=1, beta=2.0,
                kv_len=None, edgeworth=False):
    """Per-query router of ssa/gemma_ssa.py:85-131: rows qrows (B,Hq,nq,d) at positions
    pos0 + r over the complete blocks of k[:, :, :kv_len] -> (kv_num, kv_idx compact).
    `edgeworth` adds beta^2/6 <q^3, m3> to the score (ssa/gemma_ssa.py:101-102)."""
    kv_len = k.shape[2] if kv_len is None else kv_len
    mu, var, m3 = block_stats(k[:, :, :kv_len], block, "pop")
    r = scores(qrows, mu, var, 0.5 * beta, m3 if edgeworth else None, beta ** 2 / 6.0)
    return compact(select_rows(r, "query", top_c, budget_frac, local, pos0, block))


def route_query_summaries(qrows, mu, var, block, pos0, top_c=None, budget_frac=0.25, local=1,
                          beta=2.0):
    """route_query over precomputed population summaries mu, var (B, Hkv, nbk, d) of a cache
    whose blocks complete at the rows' positions are final: the per-query router of
    ssa/gemma_ssa.py:85-131 with the statistics computed once for several decode positions
    (candidates are still only the blocks complete at each position)."""
    r = scores(qrows, mu, var, 0.5 * beta)
    return compact(select_rows(r, "query", top_c, budget_frac, local, pos0, block))


def selection_gap(r64: np.ndarray, mode: str, top_c, budget_frac, query_pos=0, block=1):
    """Per row, (gap, scale): gap = (K-th best) - ((K+1)-th best) exact score among the
    candidates (inf when the row keeps all or none), scale = the row's magnitude sum used to
    bound float32 evaluation noise. A row whose gap is below a few ulps of scale may legitimately
    select differently under another float32 evaluation order (e.g. the reference's)."""
    B, Hq, R, nbk = r64.shape
    gap = np.full((B, Hq, R), np.inf)
    for i in range(R):
        cmax, keep, _ = row_geometry(mode, i, nbk, top_c, budget_frac, query_pos, block)
        k = min(keep, cmax)
        if k <= 0 or k >= cmax:
            continue
        srt = -np.sort(-r64[:, :, i, :cmax], axis=-1)
        gap[:, :, i] = srt[..., k - 1] - srt[..., k]
    return gap


def exact_scores64(rows, mu, var, coef2, m3=None, coef3=0.0):
    """fp64 scores from the same float32 operands (for gap certificates)."""
    q = rows.astype(np.float32)
    q2 = (q * q).astype(np.float32).astype(np.float64)
    Hq, Hkv = rows.shape[1], mu.shape[1]
    G = Hq // Hkv
    kh = np.arange(Hq) // G
    mu64 = mu.astype(np.float64)[:, kh]
    r = np.einsum("bhid,bhcd->bhic", q.astype(np.float64), mu64)
    mag = np.einsum("bhid,bhcd->bhic", np.abs(q.astype(np.float64)), np.abs(mu64))
    if var is not None and coef2 != 0.0:
        v64 = var.astype(np.float64)[:, kh]
        r = r + coef2 * np.einsum("bhid,bhcd->bhic", q2, v64)
        mag = mag + abs(coef2) * np.einsum("bhid,bhcd->bhic", q2, np.abs(v64))
    if m3 is not None:
        q3 = (q.astype(np.float32) ** 2 * q).astype(np.float64)
        t64 = m3.astype(np.float64)[:, kh]
        r = r + coef3 * np.einsum("bhid,bhcd->bhic", q3, t64)
        mag = mag + abs(coef3) * np.einsum("bhid,bhcd->bhic", np.abs(q3), np.abs(t64))
    return r, mag


# ---------------------------------------------------------------------------------------------
# a6 / a7: block-sparse attention (exact masked softmax)
# ---------------------------------------------------------------------------------------------


def sparse_attention(q, k, v, kv_num, kv_idx, block, scale=None, n=None, qblocks=None,
                     heads=None):
    """o_t = softmax_j(scale * q_t.k_j) v_j over keys j <= t, j < n of the selected blocks of
    t's query block -- FlexAttention with BlockMask.from_kv_blocks + mask_mod kv<=q & kv<n
    (ssa/ssa_kernel.py:33-34,125-126; ssa/gemma_ssa.py:159-162,179), in float64.
    Returns float64 (B, Hq, n, d): rows of the `heads` (default all) whose query blocks are not in
    `qblocks` (if given) are NaN; heads not in `heads` are zero. Only the rows and key heads used
    are converted to float64 (the full-size conversions dominated the cost at 131K tokens)."""
    B, Hq, N, d = q.shape
    n = N if n is None else n
    Hkv = k.shape[1]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    nb = -(-n // block)
    hs = list(range(Hq)) if heads is None else [int(h) for h in heads]
    out = np.zeros((B, Hq, n, d))
    for b in range(B):
        for h in hs:
            out[b, h] = np.nan
    for b in range(B):
        kv64 = {}
        for h in hs:
            kh = h // G
            if kh not in kv64:
                kv64 = {kh: (k[b, kh, :n].astype(np.float64), v[b, kh, :n].astype(np.float64))}
            k64, v64 = kv64[kh]
            for i in (range(nb) if qblocks is None else qblocks):
                t0, t1 = i * block, min((i + 1) * block, n)
                ids = [int(c) for c in kv_idx[b, h, i, :kv_num[b, h, i]]]
                keys = np.concatenate([np.arange(c * block, min((c + 1) * block, n)) for c in ids]) \
                    if ids else np.zeros(0, dtype=np.int64)
                s = scale * (q[b, h, t0:t1].astype(np.float64) @ k64[keys].T)
                allow = keys[None, :] <= np.arange(t0, t1)[:, None]
                s = np.where(allow, s, -np.inf)
                m = s.max(-1, keepdims=True)
                m = np.where(np.isfinite(m), m, 0.0)
                p = np.exp(s - m)
                l = p.sum(-1, keepdims=True)
                out[b, h, t0:t1] = np.where(l > 0, (p @ v64[keys]) / np.where(l > 0, l, 1), 0.0)
    return out


def dense_causal(q, k, v, scale=None):
    """Exact causal softmax attention in float64 (the full-budget special case)."""
    B, Hq, n, d = q.shape
    G = Hq // k.shape[1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    kh = np.arange(Hq) // G
    q64, k64, v64 = q.astype(np.float64), k.astype(np.float64)[:, kh], v.astype(np.float64)[:, kh]
    s = scale * np.einsum("bhtd,bhjd->bhtj", q64, k64)
    s = np.where(np.tril(np.ones((n, n), dtype=bool)), s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    return np.einsum("bhtj,bhjd->bhtd", p / p.sum(-1, keepdims=True), v64)


# ---------------------------------------------------------------------------------------------
# a10 / a11: decode
# ---------------------------------------------------------------------------------------------


def decode_attend(qvec, k, v, blocks, pos, block, scale=None):
    """One attention row over the tokens <= pos of sorted(set(blocks)), float64
    (ssa/ivf_decode.py:49-62; scale 1/sqrt(d) by default)."""
    d = qvec.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    ids = sorted(set(int(x) for x in blocks))
    idx = np.concatenate([np.arange(c * block, min((c + 1) * block, pos + 1)) for c in ids]) \
        if ids else np.zeros(0, dtype=np.int64)
    idx = idx[idx <= pos]
    if idx.size == 0:
        return np.zeros(d)
    s = scale * (k[idx].astype(np.float64) @ qvec.astype(np.float64))
    p = np.exp(s - s.max())
    return (p / p.sum()) @ v[idx].astype(np.float64)


def attend_rows(q, k, v, kv_num, kv_idx, pos0, block, scale=None):
    """Per-query rows: q (B,Hq,nq,d) at positions pos0 + r over caches k, v (B,Hkv,cap,d)."""
    B, Hq, nq, d = q.shape
    G = Hq // k.shape[1]
    out = np.zeros((B, Hq, nq, d))
    for b in range(B):
        for h in range(Hq):
            for r in range(nq):
                ids = kv_idx[b, h, r, :kv_num[b, h, r]]
                out[b, h, r] = decode_attend(q[b, h, r], k[b, h // G], v[b, h // G], ids, pos0 + r,
                                             block, scale)
    return out


# ---------------------------------------------------------------------------------------------
# f3: ssa_swap.ssa_masked (per-query routing + token-causal softmax) and its gradients
# ---------------------------------------------------------------------------------------------


def masked_route(q, k, block, top_c, local):
    """Per-query selection of ssa_masked (ssa/ssa_swap.py:36-51): key blocks zero-padded to a
    block multiple with their mean and UNBIASED variance (the zero rows count, :37-41), the
    score <q, mu> + 1/2 <q*q, var> per query row (fp32 assembly of fp64 sums), candidates = blocks
    begun at the query, top_c of them (ties to the lowest block), the own block and `local`
    predecessors. q, k (B, H, n, d) -> list-of-lists (B, H, n)."""
    B, H, n, d = q.shape
    nb = -(-n // block)
    kk = np.zeros((B, k.shape[1], nb * block, d), dtype=np.float32)
    kk[:, :, :n] = k
    mu, var, _ = block_stats(kk, block, "unbiased")
    r = scores(q.astype(np.float32), mu, var, 0.5)
    return select_rows(r, "started", top_c, 0.0, local, 0, block)


def masked_forward(q, k, v, sel, block, scale=None):
    """out (B, H, n, d) float64 and lse (B, H, n): softmax over the keys j <= i of row i's
    selected blocks of scale * q_i.k_j, times v (ssa/ssa_swap.py:52-56); query head h reads key
    head h // (H/Hkv)."""
    B, H, n, d = q.shape
    G = H // k.shape[1]
    scale = d ** -0.5 if scale is None else scale
    out = np.zeros((B, H, n, d))
    lse = np.zeros((B, H, n))
    for b in range(B):
        for h in range(H):
            K, V = k[b, h // G].astype(np.float64), v[b, h // G].astype(np.float64)
            for i in range(n):
                keys = _masked_keys(sel[b, h, i], i, block, n)
                s = scale * (K[keys] @ q[b, h, i].astype(np.float64))
                m = s.max()
                p = np.exp(s - m)
                out[b, h, i] = p @ V[keys] / p.sum()
                lse[b, h, i] = m + math.log(p.sum())
    return out, lse


def _masked_keys(blocks, i, block, n):
    return np.array([j for c in sorted(set(blocks)) for j in range(c * block, min((c + 1) * block, n))
                     if j <= i], dtype=np.int64)


def masked_grads(q, k, v, sel, g, block, scale=None):
    """Gradients of sum(out * g) through masked_forward with the selection fixed:
    P = softmax(S), dP = g V^T, dS = P (dP - rowsum(P dP)), dq = scale dS K, dk = scale dS^T q,
    dv = P^T g (float64)."""
    B, H, n, d = q.shape
    Hkv = k.shape[1]
    G = H // Hkv
    scale = d ** -0.5 if scale is None else scale
    dq = np.zeros((B, H, n, d))
    dk = np.zeros((B, Hkv, n, d))
    dv = np.zeros((B, Hkv, n, d))
    for b in range(B):
        for h in range(H):
            K, V = k[b, h // G].astype(np.float64), v[b, h // G].astype(np.float64)
            for i in range(n):
                keys = _masked_keys(sel[b, h, i], i, block, n)
                qi, gi = q[b, h, i].astype(np.float64), g[b, h, i].astype(np.float64)
                s = scale * (K[keys] @ qi)
                p = np.exp(s - s.max())
                p /= p.sum()
                dp = V[keys] @ gi
                ds = p * (dp - (p * dp).sum())
                dq[b, h, i] = scale * ds @ K[keys]
                dk[b, h // G, keys] += scale * np.outer(ds, qi)
                dv[b, h // G, keys] += np.outer(p, gi)
    return dq, dk, dv


# ---------------------------------------------------------------------------------------------
# f4: IVF router over block means (the faiss-free restatement of ssa/ivf_kernel.py:63-119)
# ---------------------------------------------------------------------------------------------


def ivf_nlist(nb: int) -> int:
    """Default list count of build_ivf (ssa/ivf_kernel.py:66): min(nb, max(4, floor(sqrt nb)))."""
    return min(nb, max(4, int(nb ** 0.5)))


def _dot_seq(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """(R, d) x (C, d) float32 -> (R, C) float32: each <a_r, b_c> accumulated in float64 in
    dimension order (a product of two float32 values is exact in float64, so every step rounds
    once, as an fma does) and rounded once to float32."""
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    acc = np.zeros((a.shape[0], b.shape[0]))
    for t in range(a.shape[1]):
        acc = acc + np.outer(a64[:, t], b64[:, t])
    return acc.astype(np.float32)


def ivf_keys(score: np.ndarray, idx) -> np.ndarray:
    """Unique uint64 ordering keys: larger score first, then the lower index."""
    idx = np.broadcast_to(np.asarray(idx, dtype=np.uint64), score.shape)
    return (score_keys(score).astype(np.uint64) << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)


def _normalised(s64: np.ndarray) -> np.ndarray:
    """fl32(s / sqrt(sum_t s_t^2)) with the squares summed in dimension order; s when zero."""
    nrm = np.add.accumulate(s64 * s64)[-1]
    return (s64 / np.sqrt(nrm) if nrm > 0 else s64).astype(np.float32)


def ivf_build(mu: np.ndarray, nlist: int, niter: int = 10):
    """One head's IVF index over its key-block means (build_ivf = faiss train + add,
    ssa/ivf_kernel.py:63-69; faiss clusters an inner-product IVF with spherical k-means).
    mu (nb, d) float32 -> (centroids (nlist, d) float32, lists: nlist ascending int64 arrays).
    Centroid c starts at the normalised mu[c * nb // nlist]; each of niter rounds assigns every
    block mean to its largest-<mu_j, c> centroid (ties to the lower c) and sets each centroid with
    members to the normalised float64 sum of its members in ascending order; a last assignment
    fills the lists. (faiss starts from a random sample and splits empty clusters; both choices
    here are deterministic instead.)"""
    nb, d = mu.shape
    m64 = mu.astype(np.float64)
    cent = np.stack([_normalised(m64[(c * nb) // nlist]) for c in range(nlist)])
    for it in range(niter + 1):
        a = ivf_keys(_dot_seq(mu, cent), np.arange(nlist)[None, :]).argmax(1)
        if it == niter:
            break
        for c in range(nlist):
            mem = np.nonzero(a == c)[0]
            if len(mem):
                s = np.add.accumulate(m64[mem], axis=0)[-1]
                if np.add.accumulate(s * s)[-1] > 0:
                    cent[c] = _normalised(s)
    return cent, [np.nonzero(a == c)[0] for c in range(nlist)]


def ivf_search(qb: np.ndarray, mu: np.ndarray, cent: np.ndarray, lists, nprobe: int,
               search_k: int, top_c: int, local: int):
    """_route_head of ssa/ivf_kernel.py:72-99 for one head: per query block i, the
    min(nprobe, nlist) lists of largest <qb_i, c>, the min(search_k, nb) members of those lists
    of largest <qb_i, mu_j> (faiss's search, :82), the first top_c of them in that order with
    j <= i (:84-85), OR blocks i-local..i (:87-89), deduplicated and ascending (:90-95).
    qb, mu (nb, d) float32 -> list of nb ascending block lists."""
    nb = mu.shape[0]
    nlist = cent.shape[0]
    npb, sk = min(nprobe, nlist), min(search_k, nb)
    ck = ivf_keys(_dot_seq(qb, cent), np.arange(nlist)[None, :])
    fine = _dot_seq(qb, mu)
    out = []
    for i in range(nb):
        probes = np.argsort(ck[i])[::-1][:npb]
        cand = np.concatenate([lists[c] for c in probes]).astype(np.int64)
        top = cand[np.argsort(ivf_keys(fine[i, cand], cand))[::-1][:sk]]
        hits = top[top <= i][:max(top_c, 0)]
        out.append(sorted(set(hits.tolist()) | set(range(max(0, i - local), i + 1))))
    return out


def ivf_route(qb: np.ndarray, mu: np.ndarray, top_c=8, local=1, nprobe=4, search_k=None,
              nlist=None, niter=10):
    """ivf_route (ssa/ivf_kernel.py:102-119) over block means: qb, mu (B, H, nb, d) ->
    (lists (B, H, nb) of ascending block lists, centroids (B, H, nlist, d), inverted lists)."""
    B, H, nb, d = mu.shape
    nlist = ivf_nlist(nb) if nlist is None else nlist
    search_k = min(2 * top_c, nb) if search_k is None else search_k
    sel = np.empty((B, H, nb), dtype=object)
    cents = np.zeros((B, H, nlist, d), dtype=np.float32)
    inv = {}
    for b in range(B):
        for h in range(H):
            cent, lists = ivf_build(mu[b, h], nlist, niter)
            cents[b, h] = cent
            inv[b, h] = lists
            for i, s in enumerate(ivf_search(qb[b, h], mu[b, h], cent, lists, nprobe, search_k,
                                             top_c, local)):
                sel[b, h, i] = s
    return sel, cents, inv


# ---------------------------------------------------------------------------------------------
# f4 (treecode): the bounded-candidate tree router of ssa/treecode.py
# ---------------------------------------------------------------------------------------------


def tree_build(k: np.ndarray, block: int, F: int = 8, top_cap: int = 8):
    """build_tree (ssa/treecode.py:34-86): k (B, H, n, d) -> list of levels from the leaves up,
    each a dict mu (BH, n_l, d) f32, var (BH, n_l, d) f32, R (BH, n_l) f32, lo (n_l,) int64.
    Leaves (:40-52): per block the mean, the population variance E[k^2] - mean^2 and R = max
    |k - fl32(mean)|; parents (:55-76): groups of F consecutive nodes (a short last group), mean
    of the child means, var mean(var_c + mu_c^2) - mean^2, R = max(|mu_c - fl32(mean)| + R_c),
    lo = min child lo; until a level holds at most top_cap nodes. Sums in float64 from the
    stored float32 values, each stored value rounded once."""
    B, H, n, d = k.shape
    BH, nb = B * H, n // block
    kb = k[:, :, :nb * block].astype(np.float64).reshape(BH, nb, block, d)
    m64 = kb.mean(axis=2)
    mu = m64.astype(np.float32)
    var = ((kb * kb).mean(axis=2) - m64 * m64).astype(np.float32)
    dev = kb - mu.astype(np.float64)[:, :, None, :]
    R = np.sqrt((dev * dev).sum(-1).max(-1)).astype(np.float32)
    levels = [dict(mu=mu, var=var, R=R, lo=np.arange(nb, dtype=np.int64) * block)]
    while levels[-1]["mu"].shape[1] > top_cap:
        ch = levels[-1]
        nc = ch["mu"].shape[1]
        npar = -(-nc // F)
        pm = np.zeros((BH, npar, d), np.float32)
        pv = np.zeros((BH, npar, d), np.float32)
        pr = np.zeros((BH, npar), np.float32)
        pl = np.zeros(npar, np.int64)
        for p in range(npar):
            c0, c1 = p * F, min(nc, p * F + F)
            cm = ch["mu"][:, c0:c1].astype(np.float64)
            m = cm.mean(axis=1)
            pm[:, p] = m.astype(np.float32)
            pv[:, p] = ((ch["var"][:, c0:c1].astype(np.float64) + cm * cm).mean(axis=1)
                        - m * m).astype(np.float32)
            dist = np.sqrt(((cm - pm[:, p].astype(np.float64)[:, None, :]) ** 2).sum(-1))
            pr[:, p] = (dist + ch["R"][:, c0:c1].astype(np.float64)).max(axis=1).astype(np.float32)
            pl[p] = ch["lo"][c0:c1].min()
        levels.append(dict(mu=pm, var=pv, R=pr, lo=pl))
    return levels


def _tree_scores(lvl, bh, nodes, q64, qn, beta):
    """Admissible bound <q, mu> + |q| R (+ beta/2 <q*q, var>) of `nodes` of head bh
    (ssa/treecode.py:98-102), float64 rounded to float32."""
    mu = lvl["mu"][bh, nodes].astype(np.float64)
    s = mu @ q64 + qn * lvl["R"][bh, nodes].astype(np.float64)
    if beta:
        s = s + 0.5 * beta * (lvl["var"][bh, nodes].astype(np.float64) @ (q64 * q64))
    return s.astype(np.float32)


def _tree_best(nodes, s32, valid, W):
    """The W best valid (node, score) pairs by (score desc, node asc), ascending by node."""
    nodes, s32 = nodes[valid], s32[valid]
    order = np.lexsort((nodes, -score_keys(s32).astype(np.int64)))[:W]
    keep = order[np.argsort(nodes[order], kind="stable")]
    return nodes[keep], s32[keep]


def tree_descend(levels, F, q: np.ndarray, W: int, top_c: int, q_pos=None, beta: float = 0.0):
    """descend_beam (ssa/treecode.py:89-137): q (BH, Q, d) -> (BH, Q, min(top_c, W)) int64 leaf
    indices, best first, -1 past the valid ones. The top level is scanned whole (:104-117), then
    each level keeps the W best valid children of the frontier (:119-133); a node whose lo
    exceeds q_pos is masked (:110-111, :130-131); ties rank by the lower node index."""
    BH, Q, d = q.shape
    tc = min(top_c, W)
    out = np.full((BH, Q, tc), -1, np.int64)
    top = len(levels) - 1
    for bh in range(BH):
        for qi in range(Q):
            q64 = q[bh, qi].astype(np.float64)
            qn = math.sqrt(float(q64 @ q64))
            qp = np.iinfo(np.int64).max if q_pos is None else int(q_pos[bh, qi])
            nodes = np.arange(levels[top]["mu"].shape[1], dtype=np.int64)
            s32 = _tree_scores(levels[top], bh, nodes, q64, qn, beta)
            fr, fs = _tree_best(nodes, s32, levels[top]["lo"][nodes] <= qp, W)
            for l in range(top - 1, -1, -1):
                nl = levels[l]["mu"].shape[1]
                ch = (fr[:, None] * F + np.arange(F)[None, :]).reshape(-1)
                ch = ch[ch < nl]
                s32 = _tree_scores(levels[l], bh, ch, q64, qn, beta)
                fr, fs = _tree_best(ch, s32, levels[l]["lo"][ch] <= qp, W)
            order = np.lexsort((fr, -score_keys(fs).astype(np.int64)))[:tc]
            out[bh, qi, :len(order)] = fr[order]
    return out


# ---------------------------------------------------------------------------------------------
# f4 (cascade): the certified causal cascade of ssa/cascade_router.py, faiss-free
# ---------------------------------------------------------------------------------------------


def _seq_sum(x64: np.ndarray, axis: int) -> np.ndarray:
    """Sum along `axis` in index order (each step rounds once, as the kernels' adds do)."""
    return np.add.accumulate(x64, axis=axis).take(-1, axis=axis)


def ccc_group_means(x: np.ndarray, group: int) -> np.ndarray:
    """(m, d) -> (m // group, d) float32: fp64 sums of each group's rows in row order, divided
    by group and rounded once (sub_block_means / block_means, ssa/cascade_router.py:46-48,
    ssa/ivf_kernel.py:50-60)."""
    m, d = x.shape
    ng = m // group
    x64 = x[:ng * group].astype(np.float32).astype(np.float64).reshape(ng, group, d)
    return (_seq_sum(x64, 1) / group).astype(np.float32)


def _sq_dist(x: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Row-wise sum over dimensions (in order) of (x - c)^2 in float64: x, c float32 (R, d)."""
    df = x.astype(np.float64) - c.astype(np.float64)
    return _seq_sum(df * df, 1)


def ccc_outliers(x: np.ndarray, means: np.ndarray, group: int, quota: int, base: int, block: int):
    """_extract_outliers (ssa/cascade_router.py:214-231): the min(quota, m) rows of largest
    fl32(||x_row - mean of its group||^2) (ties to the lower row), largest first ->
    (vectors float32, parent blocks, positions)."""
    m = x.shape[0]
    x32 = x.astype(np.float32)
    ss = _sq_dist(x32, means[np.arange(m) // group]).astype(np.float32)
    keys = ivf_keys(ss, np.arange(m))
    top = np.argsort(keys)[::-1][:min(quota, m)]
    return x32[top], (base + top) // block, base + top


def ccc_assign(X: np.ndarray, C: np.ndarray) -> np.ndarray:
    """_assign (:139-147): argmax <x, c> (fp64 dimension order, rounded), ties to the lower c."""
    return ivf_keys(_dot_seq(X, C), np.arange(C.shape[0])[None, :]).argmax(1)


def ccc_kmeans(X: np.ndarray, nlist: int, iters: int = 6, C0: np.ndarray | None = None):
    """_kmeans (:149-161): inner-product Lloyd rounds from C0 (warm) or from the evenly spaced
    rows X[c * n // nlist] (cold; the reference draws a seeded random sample); a centroid with
    members becomes fl32 of the fp64 mean of its members in ascending order."""
    n = X.shape[0]
    C = (X[[(c * n) // nlist for c in range(nlist)]] if C0 is None else C0).astype(np.float32).copy()
    X64 = X.astype(np.float64)
    for _ in range(iters):
        a = ccc_assign(X, C)
        for c in range(nlist):
            mem = np.nonzero(a == c)[0]
            if len(mem):
                C[c] = (_seq_sum(X64[mem], 0) / len(mem)).astype(np.float32)
    return C


def ccc_radii(X: np.ndarray, C: np.ndarray, a: np.ndarray, R: np.ndarray) -> np.ndarray:
    """_update_radii (:192-194): R[c] = max(R[c], fl32(||x - c||)) over the rows assigned to c."""
    r = np.sqrt(_sq_dist(X, C[a])).astype(np.float32)
    R = R.copy()
    np.maximum.at(R, a, r)
    return R


class CascadeOracle:
    """CausalCascade (ssa/cascade_router.py:66-415) on the CPU, proj = None: the state machine
    (staging, commit, first build, incremental add, rebuild), the routing metric, the
    escalation and the certificate, with the deterministic choices of the library's kernels
    (ccc_kmeans' cold start, fp64 inner products rounded once, ties to the lower index)."""

    def __init__(self, d, block=128, sub=32, top_c=8, local=1, nprobe=4, chunk_blocks=2048,
                 retrain_every=None, n_hint=None, outlier_rate=1e-3, outlier_cap=4,
                 cert_margin=0.0, max_escalations=2, escalate_factor=4, search_k=None,
                 nlist=None, kmeans=None):
        self.d, self.block, self.sub, self.spb = d, block, sub, block // sub
        self.top_c, self.local, self.nprobe = top_c, local, nprobe
        self.chunk_blocks, self.retrain_every = chunk_blocks, retrain_every
        self.outlier_rate, self.outlier_cap = outlier_rate, outlier_cap
        self.cert_margin, self.max_escalations = cert_margin, max_escalations
        self.escalate_factor = escalate_factor
        self.search_k = search_k or 4 * top_c
        if nlist is not None:
            self.nlist = nlist
        elif n_hint is not None:
            self.nlist = max(4, int((n_hint / sub) ** 0.5))
        else:
            self.nlist = None
        self.build_threshold = max(4 * (self.nlist or 4), 16384)
        self.kmeans = kmeans            # a replacement for ccc_kmeans (fixed centroids), or None
        self.means = np.zeros((0, d), np.float32)
        self.committed = 0
        self.C = None                   # centroids once the index exists
        self.Rc = None
        self.assign = None              # cell of every committed sub-mean
        self.committed_at_rebuild = 0
        self.chunks_since_rebuild = 0
        self.O = np.zeros((0, d), np.float32)
        self.O_parent = np.zeros(0, np.int64)
        self.O_pos = np.zeros(0, np.int64)

    @property
    def n_sub(self):
        return self.means.shape[0]

    def append(self, k_chunk):
        """:120-128 (commit, summarise, stage) and :214-231 (outliers)."""
        self._commit()
        k32 = np.asarray(k_chunk, np.float32)
        m = k32.shape[0]
        assert m % self.sub == 0
        mu = ccc_group_means(k32, self.sub)
        quota = max(1, int(self.outlier_rate * m))
        v, p, s = ccc_outliers(k32, mu, self.sub, quota, self.n_sub * self.sub, self.block)
        self.means = np.concatenate([self.means, mu])
        self.O = np.concatenate([self.O, v])
        self.O_parent = np.concatenate([self.O_parent, p])
        self.O_pos = np.concatenate([self.O_pos, s])

    def _commit(self):
        """:130-147."""
        if self.n_sub <= self.committed:
            return
        if self.C is None:
            self.committed = self.n_sub
            if self.n_sub >= self.build_threshold:
                self._build_index()
            return
        X = self.means[self.committed:]
        a = ccc_assign(X, self.C)
        self.assign = np.concatenate([self.assign, a])
        self.Rc = ccc_radii(X, self.C, a, self.Rc)
        self.committed = self.n_sub
        self.chunks_since_rebuild += 1
        due = (self.chunks_since_rebuild >= self.retrain_every) if self.retrain_every \
            else (self.committed >= 2 * max(1, self.committed_at_rebuild))
        if due:
            self._build_index()

    def _build_index(self, iters=6):
        """:163-190 (first build and warm rebuilds)."""
        X = self.means[:self.committed]
        if self.nlist is None:
            self.nlist = max(4, int(self.committed ** 0.5))
        if self.kmeans is not None:
            C = np.asarray(self.kmeans(X, iters), np.float32)
        else:
            warm = self.C is not None and self.C.shape[0] == self.nlist
            C = ccc_kmeans(X, self.nlist, iters, self.C if warm else None)
        self.C = C
        self.assign = ccc_assign(X, C)
        self.Rc = ccc_radii(X, C, self.assign, np.zeros(self.nlist, np.float32))
        self.committed_at_rebuild = self.committed
        self.chunks_since_rebuild = 0

    def lists(self):
        return [np.nonzero(self.assign == c)[0] for c in range(self.nlist)]

    def route(self, q_chunk, qpos, certify=False, search_k=None):
        """:282-331 -> (kv_num (nbq,), kv_idx list of ascending block lists, cert (nbq,) bool,
        rounds (nbq,))."""
        qr = ccc_group_means(np.asarray(q_chunk, np.float32), self.block)
        return self.route_rows(qr, qpos // self.block, certify, search_k)

    def route_rows(self, qr, qb_start, certify=False, search_k=None):
        nbq = qr.shape[0]
        sk0 = search_k or self.search_k
        comm = self.committed
        ns = self.n_sub - comm
        sj = np.arange(comm, self.n_sub)
        st_scores = _dot_seq(qr, self.means[comm:]) if ns else np.zeros((nbq, 0), np.float32)
        cm_scores = _dot_seq(qr, self.means[:comm]) if comm else np.zeros((nbq, 0), np.float32)
        o_scores = _dot_seq(qr, self.O) if len(self.O) else np.zeros((nbq, 0), np.float32)
        if self.C is not None:
            cs = _dot_seq(qr, self.C)
            lists = self.lists()
        kv, cert = [], np.zeros(nbq, bool)
        rounds = np.zeros(nbq, np.int32)
        for i in range(nbq):
            qblk = qb_start + i
            q64 = qr[i].astype(np.float64)
            qn = np.float32(np.sqrt(_seq_sum(q64 * q64, 0)))
            ok_st = sj // self.spb < qblk
            stk = ivf_keys(st_scores[i][ok_st], sj[ok_st])
            stk = np.sort(stk)[::-1][:min(self.search_k, ns)]
            nprobe = min(self.nprobe, self.nlist) if self.C is not None else self.nprobe
            sk = sk0
            for rnd in range(self.max_escalations + 1):
                kc = min(sk, comm)
                dlast = np.float32(-np.inf)
                cmk = np.zeros(0, np.uint64)
                probed = None
                if comm and kc:
                    if self.C is None:
                        cmk = np.sort(ivf_keys(cm_scores[i], np.arange(comm)))[::-1][:kc]
                    else:
                        ck = ivf_keys(cs[i], np.arange(self.nlist))
                        probed = np.argsort(ck)[::-1][:nprobe]
                        mem = np.concatenate([lists[c] for c in probed]).astype(np.int64)
                        cmk = np.sort(ivf_keys(cm_scores[i][mem], mem))[::-1][:kc]
                        if len(mem) >= kc:
                            dlast = _key_score(cmk[-1])
                cand = np.concatenate([cmk, stk])
                best = {}
                for key in sorted(cand.tolist(), reverse=True):         # score desc, sub asc
                    p = _key_index(key) // self.spb
                    if p not in best:
                        best[p] = key
                kept = sorted(best.items(), key=lambda t: -t[1])[:self.top_c]
                tau = _key_score(min(k for _, k in kept)) if kept else np.float32(-np.inf)
                opar = []
                cap = min(self.outlier_cap, len(self.O))
                if cap:
                    hit = np.nonzero((self.O_parent < qblk) & (o_scores[i] > tau))[0]
                    ok = np.sort(ivf_keys(o_scores[i][hit], hit))[::-1][:cap]
                    opar = [int(self.O_parent[_key_index(k)]) for k in ok.tolist()]
                loc = [qblk - L for L in range(self.local + 1) if qblk - L >= 0]
                kv_i = sorted(set([p for p, _ in kept]) | set(opar) | set(loc))
                ok_cert = False
                if certify:
                    full = len(kept) >= min(self.top_c, qblk)
                    has_tau = tau > -np.inf
                    if self.C is None:
                        ok_cert = full and (has_tau or qblk == 0)
                    else:
                        lim = np.float32(tau) - np.float32(self.cert_margin)
                        ub = cs[i] + qn * self.Rc                          # float32 ops
                        unp = np.ones(self.nlist, bool)
                        unp[probed] = False
                        mx = ub[unp].max() if unp.any() else np.float32(-np.inf)
                        ok_cert = bool(full and has_tau and mx < lim and dlast < lim)
                    rounds[i] = rnd
                if not certify or ok_cert or self.C is None:
                    break
                if rnd == self.max_escalations:
                    break
                nprobe = min(nprobe * self.escalate_factor, self.nlist)
                sk = min(sk * 2, comm)
            cert[i] = ok_cert
            kv.append(kv_i)
        return np.array([len(x) for x in kv], np.int32), kv, cert, rounds


def _key_index(key) -> int:
    return 0xFFFFFFFF - (int(key) & 0xFFFFFFFF)


def _key_score(key) -> np.float32:
    """The float32 score an ivf_keys key came from."""
    k = (int(key) >> 32) & 0xFFFFFFFF
    u = (k ^ 0x80000000) if k & 0x80000000 else (~k & 0xFFFFFFFF)
    return np.array([u], np.uint32).view(np.float32)[0]
