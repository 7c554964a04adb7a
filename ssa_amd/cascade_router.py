"""Certified causal cascade (CCC) on MI355X: the streaming chunked-causal sub-block selector of
ssa/cascade_router.py (CausalCascade :66-415, ccc_prefill :418-442) on the library's kernels
(ssa_ccc_stage / _kmeans / _index_build / _index_add / _route), with the faiss GpuIndexIVFFlat
replaced by the library's own inverted lists.

Same names, arguments and outputs as the reference module: `sub_block_means`, `CausalCascade`
(append, route -> (kv_num, kv_idx, cert or None, stats), step, and the internal _commit /
_build_index / _kmeans / _assign / _rebuild steps a test may drive or replace) and
`ccc_prefill(q, k, v, block, certify, **cfg)` -> (out, kv_num, kv_idx, cert).

Differences, all deterministic choices where the reference's are not:
  - a cold k-means starts from the evenly spaced rows X[c * n // nlist] instead of a seeded
    random sample; a centroid with members becomes fl32 of their fp64 mean;
  - inner products accumulate in fp64 in dimension order and round once to fp32, means and
    distances likewise; every ranking (search, sub-block max-pool, top_c, outliers) breaks ties
    by the lower index (faiss and torch.topk leave them unspecified);
  - outliers rank by fl32 of the squared distance to their sub-block mean (the same order as the
    reference's norm, up to fp32 ties);
  - with a projection, the routing-space sub-block means are the means of the projected keys
    (equal to the projected means up to rounding).
The selection, escalation and certificate rules are the reference's, row for row, and each
query block's escalation rounds run inside one kernel (no host round trip per round).
`res` (a faiss resources object) is accepted and ignored.
"""
from __future__ import annotations

import torch

from . import _lib
from .ssa_kernel import BLOCK, sparse_attention

NEG = float("-inf")
MAX_SEARCH = 1024   # search_k (staged, and committed after escalation) the route kernel takes
MAX_QUOTA = 2048    # outliers kept per appended chunk


def _rows(x: torch.Tensor) -> torch.Tensor:
    _lib.require_device(x)
    if x.dim() != 2:
        raise ValueError(f"expected an (n, d) tensor, got shape {tuple(x.shape)}")
    return x if x.stride(-1) == 1 else x.contiguous()


def _group_means(x: torch.Tensor, group: int) -> torch.Tensor:
    x = _rows(x)
    n, d = x.shape
    out = torch.empty(n // group, d, device=x.device, dtype=torch.float32)
    if n // group:
        _lib.call("ssa_ccc_stage", x.data_ptr(), _lib.dtype_code(x.dtype), n, d, x.stride(0), group,
                  out.data_ptr(), 0, 0, 1, None, None, None, None, 0, _lib.stream_of(x))
    return out


def sub_block_means(x: torch.Tensor, block: int = BLOCK, sub: int = 32, chunk: int = 1 << 20):
    """(n, d) -> (n // sub, d) fp32 sub-block means (ssa/cascade_router.py:46-48), fp64 sums in
    row order rounded once; `block` and `chunk` are accepted for the same call shape."""
    return _group_means(x, sub)


def _as_projectors(proj, d):
    """(project_q, project_k, d_r) as ssa/cascade_router.py:51-61: None, an object with
    project_q / project_k, or a (d, d_r) tensor applied to both (a library GEMM)."""
    if proj is None:
        return None, None, d
    if hasattr(proj, "project_q"):
        dev = torch.device("cuda", torch.cuda.current_device())
        d_r = proj.project_k(torch.zeros(1, d, device=dev)).shape[-1]
        return proj.project_q, proj.project_k, d_r
    W = proj.to("cuda").float()
    return (lambda t: t @ W), (lambda t: t @ W), W.shape[1]


class _Index:
    """The index buffer (ssa_ccc_index_size(n_cap, nlist, d) bytes) and views of its regions."""

    def __init__(self, n_cap, nlist, d, device):
        self.n_cap, self.nlist, self.d = n_cap, nlist, d
        self.bytes = int(_lib.query("ssa_ccc_index_size", n_cap, nlist, d))
        self.buf = torch.empty(self.bytes, device=device, dtype=torch.uint8)
        r = lambda x: (x + 255) // 256 * 256
        o_cent = 0
        o_rc = 2 * r(nlist * d * 4)
        o_assign = o_rc + r(nlist * 4)
        self.centroids = self.buf[o_cent:o_cent + nlist * d * 4].view(torch.float32).view(nlist, d)
        self.Rc = self.buf[o_rc:o_rc + nlist * 4].view(torch.float32)
        self.assign = self.buf[o_assign:o_assign + n_cap * 4].view(torch.int32)


class CausalCascade:
    """Streaming selector (ssa/cascade_router.py:66-415). For each chunk of `chunk_blocks`
    blocks call append(k_chunk) then route(q_chunk, qpos); ccc_prefill drives the loop."""

    def __init__(self, d, block=BLOCK, sub=32, top_c=8, local=1, nprobe=4, chunk_blocks=2048,
                 retrain_every=None, d_r=None, proj=None, n_hint=None, outlier_rate=1e-3,
                 outlier_cap=4, cert_margin=0.0, max_escalations=2, escalate_factor=4,
                 search_k=None, nlist=None, res=None, dtype=torch.float16):
        if block % sub:
            raise ValueError(f"CausalCascade: sub={sub} must divide block={block}")
        self.d, self.block, self.sub = d, block, sub
        self.spb = block // sub
        self.top_c, self.local, self.nprobe = top_c, local, nprobe
        self.chunk_blocks = chunk_blocks
        self.retrain_every = retrain_every
        self.outlier_rate, self.outlier_cap = outlier_rate, outlier_cap
        self.cert_margin, self.max_escalations = cert_margin, max_escalations
        self.escalate_factor = escalate_factor
        self.search_k = search_k or 4 * top_c
        self.dtype = dtype
        self.device = torch.device("cuda", torch.cuda.current_device())
        self.pj_q, self.pj_k, self.d_r = _as_projectors(proj, d)
        self.dr = self.d_r
        if self.d_r % 32 or self.d_r > 256:
            raise ValueError(f"CausalCascade: routing dim {self.d_r} must be a multiple of 32 "
                             "and at most 256")
        if nlist is not None:
            self.nlist = nlist
        elif n_hint is not None:
            self.nlist = max(4, int((n_hint / sub) ** 0.5))
        else:
            self.nlist = None
        self.build_threshold = max(4 * (self.nlist or 4), 16384)
        self.n_hint = n_hint
        # state
        self.means = None             # (cap, d_r) fp32 routing-space sub-means
        self.n_sub = 0
        self.committed = 0
        self.index = None             # _Index once built
        self.centroids = None         # (nlist, d_r): a view of the index
        self.Rc = None                # (nlist,) per-cell radii: a view of the index
        self.cell_of = None           # (committed,) cell of every committed sub-mean
        self.committed_at_rebuild = 0
        self.chunks_since_rebuild = 0
        self.O = None                 # (cap, d_r) fp32 outlier keys
        self.O_parent = None          # (cap,) parent block
        self.O_pos = None             # (cap,) token position
        self.n_out = 0
        self._ws = None

    # -- summaries / staging / commit ------------------------------------------------------------

    def _scratch(self, nbytes):
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = torch.empty(max(nbytes, 1 << 20), device=self.device, dtype=torch.uint8)
        return self._ws

    def _ensure_means(self, add_sub):
        need = self.n_sub + add_sub
        if self.means is None:
            cap = max(need, (self.n_hint or 0) // self.sub)
            self.means = torch.empty(cap, self.dr, device=self.device, dtype=torch.float32)
        elif need > self.means.shape[0]:
            new = torch.empty(int(need * 1.3) + 1, self.dr, device=self.device,
                              dtype=torch.float32)
            new[:self.n_sub] = self.means[:self.n_sub]
            self.means = new

    def _ensure_outliers(self, add):
        need = self.n_out + add
        if self.O is None or need > self.O.shape[0]:
            cap = max(need, int(need * 1.3) + 1,
                      int(self.outlier_rate * (self.n_hint or 0)) + 64)
            O = torch.empty(cap, self.dr, device=self.device, dtype=torch.float32)
            P = torch.empty(cap, device=self.device, dtype=torch.int64)
            S = torch.empty(cap, device=self.device, dtype=torch.int64)
            if self.n_out:
                O[:self.n_out] = self.O[:self.n_out]
                P[:self.n_out] = self.O_parent[:self.n_out]
                S[:self.n_out] = self.O_pos[:self.n_out]
            self.O, self.O_parent, self.O_pos = O, P, S

    def append(self, k_chunk):
        """Commit the previously staged chunk, then summarise and stage this one and take its
        outlier keys (ssa/cascade_router.py:120-128,214-231). k_chunk: (m, d), m a multiple of
        sub."""
        self._commit()
        k_chunk = _rows(k_chunk)
        m_tok = k_chunk.shape[0]
        if m_tok % self.sub:
            raise ValueError(f"append: {m_tok} keys are not whole sub-blocks of {self.sub}")
        m4 = m_tok // self.sub
        if m4 == 0:
            return
        kr = k_chunk if self.pj_k is None else _rows(self.pj_k(k_chunk.float()).float())
        quota = min(max(1, int(self.outlier_rate * m_tok)), m_tok)
        if quota > MAX_QUOTA:
            raise ValueError(f"append: outlier quota {quota} exceeds {MAX_QUOTA}")
        self._ensure_means(m4)
        self._ensure_outliers(quota)
        ws = self._scratch(8 * m_tok + 8 * quota * (-(-m_tok // 2048)))
        _lib.call("ssa_ccc_stage", kr.data_ptr(), _lib.dtype_code(kr.dtype), m_tok, self.dr,
                  kr.stride(0), self.sub, self.means[self.n_sub].data_ptr(), quota,
                  self.n_sub * self.sub, self.block, self.O[self.n_out].data_ptr(),
                  self.O_parent[self.n_out].data_ptr(), self.O_pos[self.n_out].data_ptr(),
                  ws.data_ptr(), ws.numel(), _lib.stream_of(kr))
        self.n_out += quota
        self.n_sub += m4

    def _commit(self):
        """Push the staged sub-means into the index, or into the flat-scanned region before the
        index exists (ssa/cascade_router.py:130-147)."""
        if self.n_sub <= self.committed:
            return
        if self.index is None:
            self.committed = self.n_sub
            if self.n_sub >= self.build_threshold:
                self._build_index()
            return
        if self.n_sub > self.index.n_cap:
            self._grow_index(self.n_sub)
        ix = self.index
        _lib.call("ssa_ccc_index_add", self.means.data_ptr(), self.committed, self.n_sub, self.dr,
                  ix.nlist, ix.buf.data_ptr(), ix.n_cap, ix.bytes, _lib.stream_of(self.means))
        self.committed = self.n_sub
        self.cell_of = ix.assign[:self.committed]
        self.chunks_since_rebuild += 1
        self._maybe_rebuild()

    def _grow_index(self, need):
        """A larger index buffer with the same centroids, lists and radii (incremental radii are
        upper bounds, so they are carried over rather than recomputed)."""
        old = self.index
        new = _Index(max(need, 2 * old.n_cap), old.nlist, self.dr, self.device)
        _lib.call("ssa_ccc_index_build", self.means.data_ptr(), self.committed, self.dr, old.nlist,
                  old.centroids.data_ptr(), new.buf.data_ptr(), new.n_cap, new.bytes,
                  _lib.stream_of(self.means))
        new.Rc.copy_(old.Rc)
        self._adopt(new)

    def _adopt(self, ix):
        self.index = ix
        self.centroids = ix.centroids
        self.Rc = ix.Rc
        self.cell_of = ix.assign[:self.committed]

    def _assign(self, X):
        """Coarse assignment: argmax <X, c> over the current centroids, ties to the lower cell
        (ssa/cascade_router.py:139-147)."""
        X = _rows(X.float())
        n = X.shape[0]
        out = torch.empty(n, device=X.device, dtype=torch.int32)
        if n:
            ws = self._scratch(int(_lib.query("ssa_ccc_index_size", n, self.nlist, self.dr)))
            _lib.call("ssa_ccc_assign", X.data_ptr(), n, self.dr, self.centroids.data_ptr(),
                      self.nlist, out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(X))
        return out.long()

    def _kmeans(self, X, iters=6):
        """Inner-product Lloyd rounds, warm-started from the current centroids (rebuilds) or from
        evenly spaced rows (cold) (ssa/cascade_router.py:149-161)."""
        X = _rows(X)
        warm = self.centroids is not None and self.centroids.shape[0] == self.nlist
        C = self.centroids.clone() if warm else torch.empty(self.nlist, self.dr,
                                                             device=X.device, dtype=torch.float32)
        ws = self._scratch(int(_lib.query("ssa_ccc_index_size", X.shape[0], self.nlist, self.dr)))
        _lib.call("ssa_ccc_kmeans", X.data_ptr(), X.shape[0], self.dr, self.nlist, iters,
                  1 if warm else 0, C.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(X))
        return C

    def _build_index(self, iters=6):
        """(Re)build the index over the committed sub-means with this build's centroids: lists of
        their assignment and exact radii (ssa/cascade_router.py:163-190)."""
        X = self.means[:self.committed]
        if self.nlist is None:
            self.nlist = max(4, int(self.committed ** 0.5))
        C = self._kmeans(X, iters).float().contiguous()
        cap = max(self.committed, (self.n_hint or 0) // self.sub)
        ix = self.index
        if ix is None or ix.nlist != self.nlist or ix.n_cap < self.committed:
            ix = _Index(cap, self.nlist, self.dr, self.device)
        if C.data_ptr() == ix.centroids.data_ptr():
            C = C.clone()
        _lib.call("ssa_ccc_index_build", X.data_ptr(), self.committed, self.dr, self.nlist,
                  C.data_ptr(), ix.buf.data_ptr(), ix.n_cap, ix.bytes, _lib.stream_of(X))
        self._adopt(ix)
        self.committed_at_rebuild = self.committed
        self.chunks_since_rebuild = 0

    def _maybe_rebuild(self):
        due = (self.chunks_since_rebuild >= self.retrain_every) if self.retrain_every \
            else (self.committed >= 2 * max(1, self.committed_at_rebuild))
        if due:
            self._rebuild()

    def _rebuild(self):
        """Warm-start recluster and exact radii (ssa/cascade_router.py:196-200)."""
        if self.index is None:
            return
        self._build_index()

    # -- routing ---------------------------------------------------------------------------------

    def _query_summaries(self, q_chunk):
        qb = _group_means(q_chunk, self.block)        # (nbq, d) block means of the queries
        return qb if self.pj_q is None else _rows(self.pj_q(qb).float())

    def route(self, q_chunk, qpos, certify=False, search_k=None):
        """Route a chunk of query blocks (ssa/cascade_router.py:282-331): returns (kv_num (nbq,),
        kv_idx (nbq, W), cert (nbq,) bool or None, stats). Rows whose certificate fails are
        searched again with escalate_factor times the lists and twice the search_k, at most
        max_escalations times."""
        sk0 = search_k or self.search_k
        qr = self._query_summaries(q_chunk)
        nbq = qr.shape[0]
        qb_start = qpos // self.block
        nb_global = qb_start + nbq
        W = max(1, min(self.top_c + self.local + 1 + self.outlier_cap, nb_global))
        dev = qr.device
        kv_num = torch.zeros(nbq, dtype=torch.int32, device=dev)
        kv_idx = torch.zeros(nbq, W, dtype=torch.int32, device=dev)
        cert = torch.zeros(nbq, dtype=torch.uint8, device=dev)
        rounds = torch.zeros(nbq, dtype=torch.int32, device=dev)
        ix = self.index
        means = self.means
        ws = None
        if ix is not None and certify and self.max_escalations > 0:
            # escalation carry: per query block the best keys of the lists probed so far, as many
            # as the last round's search_k
            sk = sk0
            for _ in range(self.max_escalations):
                sk = min(2 * sk, self.committed)
            skmax = max(min(sk0, self.committed), sk)
            ws = torch.empty(nbq * skmax, dtype=torch.int64, device=dev)
        _lib.call("ssa_ccc_route", qr.data_ptr(), nbq, qb_start, self.dr,
                  None if means is None else means.data_ptr(), self.committed, self.n_sub,
                  self.spb, None if ix is None else ix.buf.data_ptr(),
                  0 if ix is None else ix.n_cap, 0 if ix is None else ix.nlist,
                  None if self.O is None else self.O.data_ptr(),
                  None if self.O_parent is None else self.O_parent.data_ptr(), self.n_out,
                  self.top_c, self.local, self.outlier_cap, self.search_k, sk0, self.nprobe,
                  self.escalate_factor, self.max_escalations, 1 if certify else 0,
                  float(self.cert_margin), kv_num.data_ptr(), kv_idx.data_ptr(), W,
                  cert.data_ptr(), rounds.data_ptr(), None if ws is None else ws.data_ptr(),
                  0 if ws is None else 8 * ws.numel(), _lib.stream_of(qr))
        stats = {"nbq": nbq, "rounds": rounds,
                 "cert_rate": float(cert.float().mean()) if certify and nbq else None}
        return kv_num, kv_idx, (cert.bool() if certify else None), stats

    # -- decode ----------------------------------------------------------------------------------

    def step(self, q_new, k_new, v_new, kbuf, vbuf, pos):
        """One decode step (ssa/cascade_router.py:407-415): route the single query over the
        committed and staged sub-means, attend over the selected blocks."""
        from .ivf_decode import decode_attend
        q_rows = q_new.reshape(1, self.d).expand(self.block, self.d).contiguous()
        kn, ki, _, _ = self.route(q_rows, qpos=(pos // self.block) * self.block)
        blocks = ki[0, :int(kn[0])].tolist()
        return decode_attend(q_new, kbuf, vbuf, blocks, pos, self.block)


@torch.no_grad()
def ccc_prefill(q, k, v, block=BLOCK, certify=False, **cfg):
    """Chunked-causal routing assembled into one (kv_num, kv_idx) and one block-sparse attention
    call (ssa/cascade_router.py:418-442). q, k, v: (1, 1, n, d). Returns (out, kv_num (1,1,nb),
    kv_idx (1,1,nb,W), cert (nb,) bool or None)."""
    B, H, n, d = q.shape
    if B != 1 or H != 1:
        raise ValueError("ccc_prefill: single-head rig, q must be (1, 1, n, d)")
    nb = n // block
    cc = CausalCascade(d, block=block, n_hint=n, **cfg)
    W = min(cc.top_c + cc.local + 1 + cc.outlier_cap, nb)
    kv_num = torch.empty(1, 1, nb, device=q.device, dtype=torch.int32)
    kv_idx = torch.zeros(1, 1, nb, W, device=q.device, dtype=torch.int32)
    cb = cc.chunk_blocks * block
    cert_all = []
    for t in range(0, n, cb):
        e = min(n, t + cb)
        cc.append(k[0, 0, t:e])
        kn, ki, cert, _ = cc.route(q[0, 0, t:e], qpos=t, certify=certify)
        b0, b1 = t // block, e // block
        kv_num[0, 0, b0:b1] = kn
        kv_idx[0, 0, b0:b1, :ki.shape[1]] = ki
        if cert is not None:
            cert_all.append(cert)
    out = sparse_attention(q, k, v, kv_num, kv_idx, block)
    cert = torch.cat(cert_all) if cert_all else None
    return out, kv_num, kv_idx, cert
