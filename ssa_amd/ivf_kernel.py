"""IVF-routed SSA on MI355X: the sub-linear block router of ssa/ivf_kernel.py with the faiss
GpuIndexIVFFlat index replaced by the library's own IVF kernels (ssa_ivf_build / ssa_ivf_route).

Same names and call shapes as the reference module: `block_means`, `build_ivf`, `ivf_route`
(-> the compressed `(kv_num, kv_idx)` contract, W = min(top_c + local + 1, nb), pad 0) and
`ssa_flex_ivf` (route -> the block-sparse attention kernel). Differences, all deterministic
choices where faiss is not: spherical k-means starts from the evenly spaced block means
mu[c * nb / nlist] instead of a random sample, runs `niter` (default 10) rounds, and leaves a
centroid without members where it is instead of splitting a large cluster; inner products are
fp64-accumulated and ties go to the lower index. `res` (a faiss resources object) is accepted
and ignored. Heads are batched: one build and one route call cover all heads; with grouped
query heads (Hq = G * Hkv) each key head's index serves its G query heads.
"""
from __future__ import annotations

import torch

from . import _lib
from .ssa_kernel import BLOCK, block_summary, sparse_attention


def block_means(x: torch.Tensor, block: int = BLOCK, chunk: int = 1 << 20) -> torch.Tensor:
    """(..., n, d) -> (..., n // block, d) fp32 block means, fp64-accumulated on the device
    (ssa/ivf_kernel.py:50-60; `chunk` is accepted for the same call shape: no fp32 copy of x is
    made at any size). A partial tail block is dropped, as the reference's n // block does."""
    n, d = x.shape[-2:]
    nb = n // block
    if nb == 0:
        raise ValueError(f"block_means: n={n} holds no full block of {block}")
    lead = x.shape[:-2]
    x4 = x[..., :nb * block, :].reshape(-1, 1, nb * block, d)
    return block_summary(x4, block, "qmean").reshape(*lead, nb, d)


class IVFIndex:
    """The IVF index of BH heads over nb block means each: the library's index buffer plus its
    geometry. `centroids`, `list_sizes`, `list_offsets` and `list_ids` view the buffer."""

    def __init__(self, buf: torch.Tensor, BH: int, nb: int, nlist: int, d: int, nprobe: int):
        self.buf, self.BH, self.nb, self.nlist, self.d, self.nprobe = buf, BH, nb, nlist, d, nprobe

    def _region(self, offset: int, count: int, dtype: torch.dtype) -> torch.Tensor:
        return self.buf[offset:offset + 4 * count].view(dtype)

    @property
    def centroids(self) -> torch.Tensor:
        return self._region(0, self.BH * self.nlist * self.d, torch.float32).view(
            self.BH, self.nlist, self.d)

    def _offsets(self):
        r = lambda x: (x + 255) // 256 * 256
        o_count = r(self.BH * self.nlist * self.d * 4)
        o_off = o_count + r(self.BH * self.nlist * 4)
        o_ids = o_off + r(self.BH * (self.nlist + 1) * 4)
        return o_count, o_off, o_ids

    @property
    def list_sizes(self) -> torch.Tensor:
        return self._region(self._offsets()[0], self.BH * self.nlist, torch.int32).view(
            self.BH, self.nlist)

    @property
    def list_offsets(self) -> torch.Tensor:
        return self._region(self._offsets()[1], self.BH * (self.nlist + 1), torch.int32).view(
            self.BH, self.nlist + 1)

    @property
    def list_ids(self) -> torch.Tensor:
        return self._region(self._offsets()[2], self.BH * self.nb, torch.int32).view(
            self.BH, self.nb)


def default_nlist(nb: int) -> int:
    """build_ivf's list count (ssa/ivf_kernel.py:66)."""
    return min(nb, max(4, int(nb ** 0.5)))


def build_ivf(mu: torch.Tensor, nlist: int | None = None, nprobe: int = 4, res=None,
              niter: int = 10) -> IVFIndex:
    """IVF index over block means (ssa/ivf_kernel.py:63-69): mu (nb, d) or (BH, nb, d) fp32 ->
    IVFIndex with nlist lists per head (default min(nb, max(4, sqrt nb)))."""
    _lib.require_device(mu)
    mu3 = mu.reshape(-1, *mu.shape[-2:]).to(torch.float32).contiguous()
    BH, nb, d = mu3.shape
    nlist = default_nlist(nb) if nlist is None else int(nlist)
    size = int(_lib.query("ssa_ivf_index_size", BH, nb, nlist, d))
    buf = torch.empty(size, device=mu.device, dtype=torch.uint8)
    _lib.call("ssa_ivf_build", mu3.data_ptr(), BH, nb, d, nlist, int(niter), buf.data_ptr(), size,
              _lib.stream_of(mu3))
    return IVFIndex(buf, BH, nb, nlist, d, min(int(nprobe), nlist))


def search(index: IVFIndex, qb: torch.Tensor, top_c: int = 8, local: int = 1,
           nprobe: int | None = None, search_k: int | None = None):
    """Routes every query block of qb (BH * G, nb, d) through `index` (_route_head,
    ssa/ivf_kernel.py:72-99) -> (kv_num (BH * G, nb), kv_idx (BH * G, nb, W)) int32. Query head
    h searches index head h // G (G = 1: one index per head, as the reference builds)."""
    _lib.require_device(qb)
    rows = qb.numel() // (index.nb * index.d)
    if rows * index.nb * index.d != qb.numel() or rows % index.BH:
        raise ValueError(f"search: qb {tuple(qb.shape)} is not (BH*G, {index.nb}, {index.d}) "
                         f"for an index of BH={index.BH} heads")
    G = rows // index.BH
    qb = qb.reshape(rows, index.nb, index.d).to(torch.float32).contiguous()
    nb = index.nb
    nprobe = index.nprobe if nprobe is None else int(nprobe)
    search_k = min(2 * top_c, nb) if search_k is None else int(search_k)
    W = min(top_c + local + 1, nb)
    kv_num = torch.empty(rows, nb, device=qb.device, dtype=torch.int32)
    kv_idx = torch.empty(rows, nb, W, device=qb.device, dtype=torch.int32)
    _lib.call("ssa_ivf_route", index.buf.data_ptr(), qb.data_ptr(), index.BH, G, nb, index.d,
              index.nlist, nprobe, search_k, int(top_c), int(local), kv_num.data_ptr(),
              kv_idx.data_ptr(), W, _lib.stream_of(qb))
    return kv_num, kv_idx


def ivf_route(q, k, block=BLOCK, top_c=8, local=1, nprobe=4, search_k=None, res=None,
              nlist=None, niter=10):
    """(B, Hq, n, d) q, (B, Hkv, n, d) k -> (kv_num (B, Hq, nb) int32, kv_idx (B, Hq, nb, W)
    int32) for the block-sparse attention (ssa/ivf_kernel.py:102-119): one index per (b, key
    head) over that head's key block means, searched with the query block means of each query
    head it serves (Hq a multiple of Hkv; the reference has Hq = Hkv); W = min(top_c + local + 1,
    nb)."""
    B, H, n, d = q.shape
    Hkv = k.shape[1]
    if k.shape[0] != B or k.shape[2] != n or H % Hkv:
        raise ValueError("ivf_route: k must be (B, Hkv, n, d) with Hq a multiple of Hkv")
    nb = n // block
    qb = block_means(q, block).reshape(B * H, nb, d)
    mu = block_means(k, block).reshape(B * Hkv, nb, d)
    index = build_ivf(mu, nlist, nprobe, res, niter)
    kv_num, kv_idx = search(index, qb, top_c, local, nprobe,
                            min(2 * top_c, nb) if search_k is None else search_k)
    return kv_num.view(B, H, nb), kv_idx.view(B, H, nb, -1)


def ssa_flex_ivf(q, k, v, block=BLOCK, top_c=8, local=1, nprobe=4, search_k=None):
    """IVF-routed SSA inference (ssa/ivf_kernel.py:130-134): IVF route -> block-sparse causal
    attention over the routed blocks, scale 1/sqrt(d)."""
    kv_num, kv_idx = ivf_route(q, k, block, top_c, local, nprobe, search_k)
    return sparse_attention(q, k, v, kv_num, kv_idx, block)
