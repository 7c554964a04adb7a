"""The reference's CPU path restated in torch float32 -- the CPU BASELINE timed by bench.py.

TEST / BENCHMARK INFRASTRUCTURE ONLY: tests/ check it and bench.py's cpu_baseline leg times it;
nothing in ssa_amd/ imports it and it is never a fallback for the HIP kernels. Unlike the float64
NumPy oracle (ssa_oracle.py, the checker), this module runs the reference's own operator sequence
with torch on the host's cores, in the reference's dtype (float32), so that its time is what the
reference's path costs on this host's CPU:

  route_budget    ssa/ssa_kernel.py:61-119 -- view -> float -> mean / var -> einsum -> masked_fill
                  -> topk -> scatter -> local OR -> causal AND -> kv_num / argsort, on the
                  query-head-repeated keys as the model path passes them (ssa/gemma_ssa.py:196,154)
  attend_blocks   the block-sparse causal softmax of FlexAttention for chosen (head, query block)
                  pairs (ssa/ssa_kernel.py:125-126, mask_mod kv <= q): the selected blocks' keys
                  gathered, scores scaled, masked, softmax and the value product in float32
  decode_scores / decode_step
                  one decode step over resident block summaries: the score of
                  ssa/gemma_ssa.py:99-100 at q_len = 1 over the complete blocks, topk, own +
                  `local` predecessors (:104-131), then decode_attend (ssa/ivf_decode.py:49-62)
                  per query head
"""
from __future__ import annotations

import math

import torch


def _repeat_kv(x: torch.Tensor, n: int) -> torch.Tensor:
    if n == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, n, s, d).reshape(b, h * n, s, d)


@torch.no_grad()
def route_budget(q: torch.Tensor, k: torch.Tensor, block: int, top_c=None, budget_frac=0.25,
                 local=1, beta=2.0):
    """block_route_budget (ssa/ssa_kernel.py:61-119) in torch float32 on the CPU. q (B,Hq,n,d),
    k (B,Hkv,n,d) with n a block multiple; k is repeated to Hq heads first. Returns
    (kv_num (B,Hq,nb) int32, kv_idx (B,Hq,nb,nb) int32 in argsort order, sel bool)."""
    B, H, n, d = q.shape
    k = _repeat_kv(k, H // k.shape[1])
    nb = n // block
    ks = k.reshape(B, H, nb, block, d).float()
    qb = q.reshape(B, H, nb, block, d).float().mean(3)
    mu = ks.mean(3)
    var = ks.var(3, unbiased=False)
    r = (torch.einsum("bhqd,bhcd->bhqc", qb, mu)
         + 0.5 * beta * torch.einsum("bhqd,bhcd->bhqc", qb * qb, var))
    qi = torch.arange(nb)
    routable = qi[:, None] > qi[None, :]
    r = r.masked_fill(~routable[None, None], float("-inf"))
    nvis = routable.sum(-1)
    keep = (torch.full_like(nvis, top_c) if top_c is not None
            else torch.clamp((budget_frac * nvis.float()).ceil().long(), min=1))
    top = max(1, min(int(keep.max().item()), nb))
    sel = torch.zeros(B, H, nb, nb, dtype=torch.bool)
    idx = r.topk(top, dim=-1).indices
    keep_mask = torch.arange(top)[None, :] < keep[:, None]
    sel.scatter_(-1, idx, keep_mask[None, None].expand(B, H, nb, top))
    causal = qi[:, None] >= qi[None, :]
    for lag in range(local + 1):
        sel |= (qi[:, None] - lag == qi[None, :])[None, None] & causal[None, None]
    sel &= causal[None, None]
    kv_num = sel.sum(-1).to(torch.int32)
    kv_idx = torch.argsort(sel.int(), dim=-1, descending=True, stable=True).to(torch.int32)
    return kv_num, kv_idx, sel


@torch.no_grad()
def attend_blocks(q, k, v, kv_num, kv_idx, block: int, pairs, scale=None):
    """Block-sparse causal attention of the given (head, query block) pairs: query rows of block
    i of head h attend the keys j <= t of blocks kv_idx[0, h, i, :kv_num[0, h, i]] (float32
    softmax, the output in q's dtype). Returns {(h, i): out (rows, d)}."""
    B, Hq, n, d = q.shape
    G = Hq // k.shape[1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = {}
    for h, i in pairs:
        ids = kv_idx[0, h, i, :int(kv_num[0, h, i])].long()
        rows = (ids[:, None] * block + torch.arange(block)[None, :]).reshape(-1)
        rows = rows[rows < n]
        ks = k[0, h // G].index_select(0, rows).float()
        vs = v[0, h // G].index_select(0, rows).float()
        q0 = i * block
        qs = q[0, h, q0:min(n, q0 + block)].float()
        s = (qs @ ks.T) * scale
        s = s.masked_fill(rows[None, :] > torch.arange(q0, q0 + qs.shape[0])[:, None],
                          float("-inf"))
        out[(h, i)] = (torch.softmax(s, dim=-1) @ vs).to(q.dtype)
    return out


@torch.no_grad()
def decode_scores(qrows, mu, var, beta=2.0):
    """The per-query cumulant score of ssa/gemma_ssa.py:99-100 at q_len = 1: qrows (Hq, d) against
    resident summaries mu, var (Hkv, nbk, d) -> (Hq, nbk) float32."""
    Hq, d = qrows.shape
    G = Hq // mu.shape[0]
    q = qrows.float().reshape(mu.shape[0], G, d)
    r = (torch.einsum("hgd,hcd->hgc", q, mu) + 0.5 * beta * torch.einsum("hgd,hcd->hgc", q * q, var))
    return r.reshape(Hq, -1)


@torch.no_grad()
def decode_step(qrows, kcache, vcache, mu, var, pos: int, block: int, top_c: int, local: int,
                beta=2.0):
    """One routed decode step for the query rows (Hq, d) at position `pos` over caches
    (Hkv, cap, d) whose complete blocks' summaries are mu, var: route (top_c of the blocks
    complete at pos, own + `local` predecessors) and decode_attend each head. Returns
    (out (Hq, d) in the cache dtype, the selected block lists)."""
    Hq, d = qrows.shape
    G = Hq // kcache.shape[0]
    ncomp = (pos + 1) // block
    r = decode_scores(qrows, mu[:, :ncomp], var[:, :ncomp], beta)
    own = pos // block
    picks = (r.topk(min(top_c, ncomp), dim=-1).indices if ncomp
             else torch.zeros(Hq, 0, dtype=torch.long))
    outs, lists = [], []
    for h in range(Hq):
        blocks = set(picks[h].tolist()) | {c for c in range(own - local, own + 1) if c >= 0}
        ids = sorted(blocks)
        idx = torch.cat([torch.arange(c * block, min((c + 1) * block, pos + 1)) for c in ids])
        ks = kcache[h // G].index_select(0, idx).float()
        vs = vcache[h // G].index_select(0, idx).float()
        w = torch.softmax((qrows[h].float() @ ks.T) / math.sqrt(d), dim=-1)
        outs.append((w @ vs).to(kcache.dtype))
        lists.append(ids)
    return torch.stack(outs), lists
