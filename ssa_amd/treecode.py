"""Treecode router on MI355X: the bounded-candidate sub-linear block selector of ssa/treecode.py
(build_tree, descend_beam) on the library's kernels (ssa_tree_build / ssa_tree_descend).

Same names and call shapes as the reference module: `TreeLevel`, `build_tree(k, block, F,
top_cap)` -> (levels, F) and `descend_beam(levels, F, q, W, top_c, q_pos, beta)` -> (BH, Q,
min(top_c, W)) leaf-block indices (int64, best first, -1 = empty), plus `tree_router` (the
reference benchmark's Q-tiled descent, ssa/treecode_bench.py:35-37) and `tree_route`, the
compact (kv_num, kv_idx) contract of the block-sparse attention for causal query-block routing.
Differences, all deterministic where the reference's float32 torch code is not: statistics and
scores are accumulated in float64 and rounded once to float32, and ties rank by the lower node
index at every level (torch.topk leaves them unspecified). The levels are views into one device
buffer; descend_beam takes the levels build_tree returned.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from .ssa_kernel import BLOCK

MAX_W, MAX_F, MAX_TOP_CAP = 64, 16, 64


@dataclass
class TreeLevel:
    """One level of the tree (ssa/treecode.py:25-31), views into the tree buffer."""
    mu: torch.Tensor   # (BH, n_l, d) node means
    R: torch.Tensor    # (BH, n_l) recursive radii
    var: torch.Tensor  # (BH, n_l, d) diagonal variance (cumulant term)
    lo: torch.Tensor   # (n_l,) earliest token index in the node's span
    n: int             # node count at this level


class TreeLevels(list):
    """The levels of build_tree (leaves first) with the buffer and geometry the kernels read."""

    def __init__(self, levels, buf, BH, nb, d, F, top_cap):
        super().__init__(levels)
        self.buf, self.BH, self.nb, self.d, self.F, self.top_cap = buf, BH, nb, d, F, top_cap


def _layout(BH, nb, d, F, top_cap):
    """Per level (n, mu, var, R, lo byte offsets), as tree.hip lays the buffer out."""
    r = lambda x: (x + 255) // 256 * 256
    out, off, n = [], 0, nb
    while True:
        o_mu = off
        off += r(BH * n * d * 4)
        o_var = off
        off += r(BH * n * d * 4)
        o_r = off
        off += r(BH * n * 4)
        o_lo = off
        off += r(n * 8)
        out.append((n, o_mu, o_var, o_r, o_lo))
        if n <= top_cap:
            break
        n = -(-n // F)
    return out, off


@torch.no_grad()
def build_tree(k: torch.Tensor, block: int = BLOCK, F: int = 8, top_cap: int = 8):
    """k: (B, H, n, d) -> (levels, F): levels[0] = the n // block leaf key blocks, ascending to
    the (<= top_cap node) top (ssa/treecode.py:34-86)."""
    _lib.require_device(k)
    if k.dim() != 4:
        raise ValueError("build_tree: k must be (B, H, n, d)")
    if k.stride(-1) != 1:
        k = k.contiguous()
    B, H, n, d = k.shape
    nb = n // block
    if nb < 1:
        raise ValueError(f"build_tree: n={n} holds no whole block of {block}")
    if not 2 <= F <= MAX_F or not 1 <= top_cap <= MAX_TOP_CAP:
        raise ValueError(f"build_tree: need 2 <= F <= {MAX_F} and 1 <= top_cap <= {MAX_TOP_CAP}")
    BH = B * H
    size = int(_lib.query("ssa_tree_size", BH, nb, d, F, top_cap))
    if size == 0:
        raise ValueError("build_tree: unsupported geometry")
    buf = torch.empty(size, device=k.device, dtype=torch.uint8)
    strides = _lib.i64_array([k.stride(0), k.stride(1), k.stride(2)])
    _lib.call("ssa_tree_build", k.data_ptr(), _lib.dtype_code(k.dtype), B, H, n, d, block, strides,
              F, top_cap, buf.data_ptr(), size, _lib.stream_of(k))
    lay, total = _layout(BH, nb, d, F, top_cap)
    if total != size:
        raise RuntimeError("build_tree: tree layout disagrees with the library's")
    levels = []
    for nl, o_mu, o_var, o_r, o_lo in lay:
        f32 = lambda o, cnt: buf[o:o + 4 * cnt].view(torch.float32)
        levels.append(TreeLevel(mu=f32(o_mu, BH * nl * d).view(BH, nl, d),
                                R=f32(o_r, BH * nl).view(BH, nl),
                                var=f32(o_var, BH * nl * d).view(BH, nl, d),
                                lo=buf[o_lo:o_lo + 8 * nl].view(torch.int64), n=nl))
    return TreeLevels(levels, buf, BH, nb, d, F, top_cap), F


def _descend(levels, F, q, W, top_c, q_pos=None, beta=0.0):
    """descend_beam's selections as the kernel writes them: int32, -1 = empty."""
    if not isinstance(levels, TreeLevels):
        raise TypeError("descend_beam: levels must come from ssa_amd.treecode.build_tree")
    if F != levels.F:
        raise ValueError(f"descend_beam: the tree was built with F={levels.F}, not {F}")
    _lib.require_device(q)
    BH, Q, d = q.shape
    if BH != levels.BH or d != levels.d:
        raise ValueError(f"descend_beam: q {tuple(q.shape)} does not match the tree "
                         f"(BH={levels.BH}, d={levels.d})")
    W, top_c = int(W), int(top_c)
    if not 1 <= W <= MAX_W or W * F > 1024 or top_c < 1:
        raise ValueError(f"descend_beam: need 1 <= W <= {MAX_W}, W*F <= 1024, top_c >= 1")
    qf = q.to(torch.float32).contiguous()
    qp = None
    if q_pos is not None:
        qp = q_pos.to(device=q.device, dtype=torch.int64).expand(BH, Q).contiguous()
    tc = min(top_c, W)
    sel = torch.empty(BH, Q, tc, device=q.device, dtype=torch.int32)
    _lib.call("ssa_tree_descend", levels.buf.data_ptr(), qf.data_ptr(),
              0 if qp is None else qp.data_ptr(), BH, Q, levels.nb, d, F, levels.top_cap, W,
              top_c, float(beta), sel.data_ptr(), _lib.stream_of(qf))
    return sel


@torch.no_grad()
def descend_beam(levels, F, q, W, top_c, q_pos=None, beta=0.0):
    """q: (BH, Q, d). Returns (BH, Q, min(top_c, W)) leaf-block indices (-1 = empty), best first;
    fixed beam width W (ssa/treecode.py:89-137)."""
    return _descend(levels, F, q, W, top_c, q_pos, beta).long()


def tree_router(levels, F, qb, W, top_c, tile=4096):
    """The reference benchmark's router (ssa/treecode_bench.py:35-37): descend_beam over qb
    (BH, nq, d) in tiles of `tile` query rows, concatenated."""
    return torch.cat([descend_beam(levels, F, qb[:, i:i + tile], W, top_c)
                      for i in range(0, qb.shape[1], tile)], dim=1)


@torch.no_grad()
def tree_route(q, k, block=BLOCK, top_c=8, local=1, W=16, F=8, top_cap=8, beta=0.0):
    """Causal query-block routing through the tree, in the block-sparse attention's compact
    contract: q (B, Hq, n, d), k (B, Hkv, n, d) -> (kv_num (B, Hq, nb), kv_idx (B, Hq, nb, W'))
    int32, W' = min(top_c, W) + local + 1. Query block i descends its key head's tree with the
    block mean of its queries and q_pos = i * block (a node whose first token lies after the
    query block's first token is masked, so every leaf it selects is a block <= i); its list is
    the selected leaves OR blocks i - local .. i, ascending."""
    from .ssa_kernel import block_summary
    B, Hq, n, d = q.shape
    Hkv = k.shape[1]
    if k.shape[0] != B or k.shape[2] != n or Hq % Hkv:
        raise ValueError("tree_route: k must be (B, Hkv, n, d) with Hq a multiple of Hkv")
    G = Hq // Hkv
    nb = n // block
    levels, _ = build_tree(k[:, :, :nb * block], block, F, top_cap)
    qb = block_summary(q[:, :, :nb * block], block, "qmean").view(B, Hkv, G, nb, d)
    qb = qb.reshape(B * Hkv, G * nb, d)
    pos = (torch.arange(nb, device=q.device, dtype=torch.int64) * block).repeat(G)
    sel = _descend(levels, F, qb, W, top_c, q_pos=pos.expand(B * Hkv, G * nb), beta=beta)
    # rows (b, kv head, g, i) are rows (b, h = kv head * G + g, i)
    tc = sel.shape[-1]
    Wp = tc + local + 1
    kv_num = torch.empty(B, Hq, nb, device=q.device, dtype=torch.int32)
    kv_idx = torch.empty(B, Hq, nb, Wp, device=q.device, dtype=torch.int32)
    _lib.call("ssa_tree_pack", sel.data_ptr(), B * Hq * nb, nb, tc, local, kv_num.data_ptr(),
              kv_idx.data_ptr(), Wp, _lib.stream_of(sel))
    return kv_num, kv_idx
