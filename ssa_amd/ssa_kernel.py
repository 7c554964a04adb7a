"""Drop-in for the reference's routed block-sparse prefill (ssa/ssa_kernel.py), on gfx950 HIP kernels.

Same names, arguments and return values as the reference:

    block_route(q, k, block, top_c, local, routing)              ssa/ssa_kernel.py:37-58
    block_route_budget(q, k, block, budget_frac, top_c, local,
                       beta, edgeworth, n_real, sub, proj)       ssa/ssa_kernel.py:61-119
    ssa_flex(q, k, v, block, top_c, local, routing)              ssa/ssa_kernel.py:122-126
    dense(q, k, v)                                               ssa/ssa_kernel.py:129-130

plus the primitives they are built from (block_summary, route, sparse_attention). Every call is
asynchronous on the current stream (no host synchronisation, unlike the reference's `.item()` at
ssa/ssa_kernel.py:107). Differences by design:
  * K/V may have fewer heads than Q (GQA: query head h reads key head h // (Hq/Hkv)); the
    reference needs repeat_kv copies (ssa/gemma_ssa.py:58-63).
  * Routers return the dense `sel` and argsort-order `kv_idx` of the reference by default;
    `compact=True` returns (kv_num, kv_idx[..., :W], None), the form the attention consumes.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import _lib

BLOCK = 128


# ---------------------------------------------------------------------------------------------
# primitives
# ---------------------------------------------------------------------------------------------

def _bhn_strides(t: torch.Tensor) -> tuple[int, int, int]:
    if t.dim() != 4:
        raise ValueError(f"expected a (B, H, n, d) tensor, got shape {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise ValueError("the head dimension must be contiguous")
    return t.stride(0), t.stride(1), t.stride(2)


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Returns t, or a contiguous copy when its layout violates the kernels' 16-byte rules."""
    vec = 4 if t.dtype == torch.float32 else 8
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s % vec == 0 for s in t.stride()[:-1])
    return t if ok else t.contiguous()


def block_summary(x: torch.Tensor, block: int, mode: str = "pop", n_real: int | None = None,
                  with_m3: bool = False):
    """Per-block summaries of x (B, H, n, d) -> fp32 (B, H, ceil(n/block), d) tensors.

    mode "pop": (mu, var, m3|None) over rows < n_real (ssa/ssa_kernel.py:80-91,
    ssa/gemma_ssa.py:65-82; n_real > n counts rows [n, n_real) as zeros, the padding of
    ssa/ssa_swap.py:37-41); "unbiased": (mu, var) with var/(cnt-1) (ssa/ssa_kernel.py:43,47);
    "qmean": the query-block mean sum(rows)/block (ssa/ssa_kernel.py:44,79).
    """
    if torch.compiler.is_compiling():
        from . import torch_ops as T
        if mode == "qmean":
            return T.block_qmean(x, block)
        mu, var, m3 = T.block_stats(x, block, mode == "unbiased",
                                    -1 if n_real is None else int(n_real), bool(with_m3))
        return mu, var, (m3 if with_m3 else None)
    return _block_summary_impl(x, block, mode, n_real, with_m3)


def _block_summary_impl(x, block, mode, n_real, with_m3):
    _lib.require_device(x)
    x = _aligned(x)
    B, H, n, d = x.shape
    nb = -(-n // block)
    code = {"pop": _lib.STATS_POP, "unbiased": _lib.STATS_UNBIASED, "qmean": _lib.STATS_QMEAN}[mode]
    mu = torch.empty(B, H, nb, d, device=x.device, dtype=torch.float32)
    var = None if mode == "qmean" else torch.empty_like(mu)
    m3 = torch.empty_like(mu) if (with_m3 and mode != "qmean") else None
    sb, sh, sn = _bhn_strides(x)
    _lib.call("ssa_block_summary", x.data_ptr(), _lib.dtype_code(x.dtype), B, H, n, d, sb, sh, sn,
              block, n if n_real is None else int(n_real), code, _lib.ptr(mu), _lib.ptr(var),
              _lib.ptr(m3), _lib.stream_of(x))
    if mode == "qmean":
        return mu
    return mu, var, m3


_ROUTE_MODES = {"budget": _lib.ROUTE_BUDGET, "flat": _lib.ROUTE_FLAT, "query": _lib.ROUTE_QUERY,
                "started": _lib.ROUTE_STARTED}


def route_width(mode: str, nbq: int, nbk: int, top_c: int | None, budget_frac: float,
                local: int, query_pos: int = 0, block: int = 1) -> int:
    return int(_lib.query("ssa_route_width", _ROUTE_MODES[mode], nbq, nbk,
                          -1 if top_c is None else int(top_c), float(budget_frac), int(local),
                          int(query_pos), int(block)))


# Largest router workspace the wrappers allocate (score keys, tile bounds, split operands): rows
# beyond it are routed in chunks. 4 GiB (1.4 % of an MI355X's HBM) routes a 12.6 M-token head
# (49,152 blocks) in 3 chunks; at 1 GiB it takes 10 and ~7 % longer.
ROUTE_WORKSPACE_LIMIT = 4 << 30


def route(rows: torch.Tensor, mu: torch.Tensor, var: torch.Tensor | None, m3: torch.Tensor | None,
          mode: str, top_c: int | None, budget_frac: float, local: int, coef2: float,
          coef3: float = 0.0, query_pos: int = 0, block: int = 1,
          workspace_limit: int = ROUTE_WORKSPACE_LIMIT, pool: int = 1):
    """Cumulant router over precomputed summaries -> compact (kv_num, kv_idx).

    rows (B, Hq, nbq, d) fp32, fp16 or bf16 (16-bit rows are read as their exact fp32 values, so
    a 16-bit q needs no fp32 copy): query-block means (mode "budget"/"flat") or query vectors
    ("query": blocks complete at position query_pos + r; "started": blocks begun there, own
    included). mu/var/m3 (B, Hkv, nbk*pool, d) fp32:
    with pool > 1 they are sub-block summaries and a key block scores as the max of its pool
    sub-blocks (ssa/ssa_kernel.py:100). Returns kv_num (B, Hq, nbq) int32 and
    kv_idx (B, Hq, nbq, W) int32 (ascending, padded 0).
    """
    if torch.compiler.is_compiling():
        from . import torch_ops as T
        return T.route(rows, mu, var, m3, mode, -1 if top_c is None else int(top_c),
                       float(budget_frac), int(local), float(coef2), float(coef3),
                       int(query_pos), int(block), int(pool))
    return _route_impl(rows, mu, var, m3, mode, top_c, budget_frac, local, coef2, coef3,
                       query_pos, block, workspace_limit, pool)


def _route_impl(rows, mu, var, m3, mode, top_c, budget_frac, local, coef2, coef3, query_pos,
                block, workspace_limit=ROUTE_WORKSPACE_LIMIT, pool=1):
    _lib.require_device(rows, mu, var, m3)
    B, Hq, nbq, d = rows.shape
    Hkv, nbs = mu.shape[1], mu.shape[2]
    if pool < 1 or nbs % pool:
        raise ValueError(f"route: {nbs} summaries are not a multiple of pool={pool}")
    nbk = nbs // pool
    rows, mu = rows.contiguous(), mu.contiguous()
    var = None if var is None else var.contiguous()
    m3 = None if m3 is None else m3.contiguous()
    W = route_width(mode, nbq, nbk, top_c, budget_frac, local, query_pos, block)
    dev = rows.device
    kv_num = torch.empty(B, Hq, nbq, device=dev, dtype=torch.int32)
    kv_idx = torch.empty(B, Hq, nbq, W, device=dev, dtype=torch.int32)
    # every row in one pass with the operands split once (ssa_route_workspace_size_split) when it
    # fits the limit, else the limit (rows routed in chunks), at least one row's keys
    nterms = 1 + (var is not None) + (m3 is not None)
    full = int(_lib.query("ssa_route_workspace_size_split", B, Hq, Hkv, nbq, nbs, d, nterms))
    per_i = int(_lib.query("ssa_route_workspace_size", B, Hq, 1, nbs))
    ws_bytes = max(per_i, min(full, workspace_limit))
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8)
    _lib.call("ssa_route_pooled", rows.data_ptr(), _lib.dtype_code(rows.dtype), mu.data_ptr(),
              _lib.ptr(var), _lib.ptr(m3), B,
              Hq, Hkv, nbq, nbk, int(pool), d, _ROUTE_MODES[mode],
              -1 if top_c is None else int(top_c), float(budget_frac), int(local), float(coef2),
              float(coef3), int(query_pos), int(block), kv_num.data_ptr(), kv_idx.data_ptr(), W,
              ws.data_ptr(), ws_bytes, _lib.stream_of(rows))
    return kv_num, kv_idx


def project_rows(x: torch.Tensor, w) -> torch.Tensor:
    """x (..., din) fp32 @ w (din, dout) -> (..., dout) fp32, accumulated in fp64 and rounded once
    (the projections of ssa/ssa_kernel.py:92-94)."""
    _lib.require_device(x)
    w = torch.as_tensor(w, dtype=torch.float32, device=x.device).contiguous()
    din, dout = w.shape
    if x.shape[-1] != din:
        raise ValueError(f"project_rows: x has {x.shape[-1]} columns, w has {din} rows")
    xc = x.float().contiguous()
    rows = xc.numel() // din
    out = torch.empty(*x.shape[:-1], dout, device=x.device, dtype=torch.float32)
    _lib.call("ssa_project_rows", xc.data_ptr(), w.data_ptr(), rows, din, dout, out.data_ptr(),
              _lib.stream_of(x))
    return out


def expand_selection(kv_num: torch.Tensor, kv_idx: torch.Tensor, nbk: int):
    """Compact lists -> the reference's dense (kv_idx (…, nbk) in argsort order, sel bool)."""
    _lib.require_device(kv_num, kv_idx)
    lead = kv_num.shape
    W = kv_idx.shape[-1]
    rows = kv_num.numel()
    sel = torch.empty(*lead, nbk, device=kv_num.device, dtype=torch.uint8)
    full = torch.empty(*lead, nbk, device=kv_num.device, dtype=torch.int32)
    _lib.call("ssa_expand_selection", kv_num.contiguous().data_ptr(),
              kv_idx.contiguous().data_ptr(), rows, W, nbk, sel.data_ptr(), full.data_ptr(),
              _lib.stream_of(kv_num))
    return full, sel.view(torch.bool)


def transpose_v(v: torch.Tensor, block: int) -> torch.Tensor:
    """V (B, Hkv, n, d) 16-bit, d in 64 / 128 / 256 / 512 -> the V^T workspace (B, Hkv, d,
    ceil(n/block)*block) that the 16-bit attention kernels read (keys >= n zero-filled). Pass it
    to sparse_attention(vt=...) to skip the per-call transpose."""
    _lib.require_device(v)
    v = _aligned(v)
    B, Hkv, n, d = v.shape
    dt = _lib.dtype_code(v.dtype)
    nbytes = int(_lib.query("ssa_sparse_attn_workspace_size", dt, B, Hkv, n, d, block))
    n_pad = -(-n // block) * block
    # the whole attention workspace (V^T first, then the kernel's per-tile key-norm maxima),
    # returned as its V^T view
    ws = torch.empty(nbytes, device=v.device, dtype=torch.uint8)
    vt = ws[:B * Hkv * d * n_pad * v.element_size()].view(v.dtype).view(B, Hkv, d, n_pad)
    _lib.call("ssa_transpose_v", v.data_ptr(), dt, B, Hkv, n, d, block, *_bhn_strides(v),
              vt.data_ptr(), nbytes, _lib.stream_of(v))
    return vt


class PreparedKV:
    """The per-(k, v) part of one sparse_attention call (ssa_sparse_attn_prepare): V^T and, at
    head dim 64, the fp16 key copy, per-tile key-norm maxima and cleared flags, in the call's
    workspace. Built by prepare_attention, consumed by one sparse_attention(prepared=...) call."""

    def __init__(self, ws, shape, dtype, block, device):
        self.ws, self.shape, self.dtype, self.block, self.device = ws, shape, dtype, block, device
        self.used = False


def prepare_attention(k: torch.Tensor, v: torch.Tensor, block: int,
                      workspace: torch.Tensor | None = None) -> PreparedKV:
    """k, v (B, Hkv, n, d) 16-bit -> the PreparedKV of one sparse_attention call on them, written
    on the current stream. It depends on k and v only, so it can run on a second stream while the
    router (which needs q and the key summaries) runs on the first; the attention call then skips
    that pass. Head dims 64 / 128 / 256 / 512, block 64 or a multiple of 128.
    `workspace`: a uint8 device buffer of at least ssa_sparse_attn_workspace_size bytes to write
    into (e.g. one buffer reused step after step, no allocation per call); the caller orders this
    call after the previous attention call that read it."""
    _lib.require_device(k, v)
    if k.dtype != v.dtype or k.shape != v.shape or k.dim() != 4:
        raise ValueError("prepare_attention: k and v must be (B, Hkv, n, d) of one dtype")
    k, v = _aligned(k), _aligned(v)
    B, Hkv, n, d = k.shape
    dt = _lib.dtype_code(k.dtype)
    nbytes = int(_lib.query("ssa_sparse_attn_workspace_size", dt, B, Hkv, n, d, block))
    if workspace is None:
        ws = torch.empty(max(nbytes, 16), device=k.device, dtype=torch.uint8)
    else:
        if (workspace.dtype != torch.uint8 or workspace.device != k.device
                or not workspace.is_contiguous() or workspace.numel() < nbytes):
            raise ValueError(f"prepare_attention: workspace must be a contiguous uint8 tensor of "
                             f">= {nbytes} bytes on {k.device}")
        ws = workspace
    strides = _lib.i64_array([*_bhn_strides(k), *_bhn_strides(v)])
    _lib.call("ssa_sparse_attn_prepare", k.data_ptr(), v.data_ptr(), dt, B, Hkv, n, d, block,
              strides, ws.data_ptr(), nbytes, _lib.stream_of(k))
    return PreparedKV(ws, (B, Hkv, n, d), k.dtype, block, k.device)


def sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_num: torch.Tensor,
                     kv_idx: torch.Tensor, block: int, scale: float | None = None,
                     out: torch.Tensor | None = None, return_lse: bool = False,
                     vt: torch.Tensor | None = None, rotate: bool = False, exact: bool = False,
                     prepared: PreparedKV | None = None):
    """Block-sparse causal attention on the compact contract (replaces FlexAttention with
    BlockMask.from_kv_blocks + mask_mod kv<=q & kv<n; ssa/ssa_kernel.py:125-126,
    ssa/gemma_ssa.py:159-162,179).

    q (B, Hq, n, d); k, v (B, Hkv, n, d); kv_num (B, Hq, nb); kv_idx (B, Hq, nb, W).
    `out` may be any (B, Hq, n, d) view with a contiguous last dim (e.g. a transpose of a
    (B, n, Hq, d) buffer). `vt` is an optional V^T from transpose_v(v, block).
    Every query block walks its key blocks in list order (bit-identical outputs across calls).
    `rotate` (16-bit, head dim 64, lists of <= 128 entries; ignored under
    torch.use_deterministic_algorithms(True)): each workgroup starts its walk at a position taken
    from the GPU clock, so workgroups resident together read the same key blocks at the same
    time -- more L2 hits, outputs that vary between calls by fp32 rounding.
    `exact`: every row takes the exact running-max softmax on fp32-scaled scores (by default rows
    whose scores provably stay within +-32 log2 units take the bounded-row path, which rounds
    q*scale*log2e to fp16 for the QK product).
    `prepared`: prepare_attention(k, v, block) of these k and v (not yet used by another call);
    the call then skips its V^T / key-norm pass.
    Returns out (and lse (B, Hq, n) fp32 if requested).
    """
    if torch.compiler.is_compiling():  # V^T is rebuilt inside the op (vt is a cache only)
        from . import torch_ops as T
        sc = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
        if return_lse:
            o, lse = T.sparse_attention_lse(q, k, v, kv_num, kv_idx, int(block), sc)
        else:
            o, lse = T.sparse_attention(q, k, v, kv_num, kv_idx, int(block), sc), None
        if out is not None:
            out.copy_(o)
            o = out
        return (o, lse) if return_lse else o
    return _sparse_attention_impl(q, k, v, kv_num, kv_idx, block, scale, out, return_lse, vt,
                                  rotate, exact, prepared)


def _sparse_attention_impl(q, k, v, kv_num, kv_idx, block, scale=None, out=None,
                           return_lse=False, vt=None, rotate=False, exact=False, prepared=None):
    _lib.require_device(q, k, v, kv_num, kv_idx)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share a dtype")
    q, k, v = _aligned(q), _aligned(k), _aligned(v)
    B, Hq, n, d = q.shape
    Hkv = k.shape[1]
    if k.shape != (B, Hkv, n, d) or v.shape != k.shape:
        raise ValueError(f"k/v shape {tuple(k.shape)} incompatible with q {tuple(q.shape)}")
    nb = -(-n // block)
    if kv_num.shape != (B, Hq, nb) or kv_idx.dim() != 4 or kv_idx.shape[:3] != (B, Hq, nb):
        raise ValueError("kv_num/kv_idx shapes do not match (B, Hq, ceil(n/block)[, W])")
    if out is None:
        out = torch.empty_like(q, memory_format=torch.contiguous_format)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    kv_num = kv_num.to(torch.int32).contiguous()
    kv_idx = kv_idx.to(torch.int32).contiguous()
    tiled = TILED_HEAD_DIMS_F32 if q.dtype == torch.float32 else TILED_HEAD_DIMS
    if d not in tiled or not (block == 64 or block % 128 == 0):
        if return_lse:
            raise NotImplementedError(f"sparse_attention: return_lse needs head_dim in "
                                      f"{tiled} and block 64 or a multiple of 128, "
                                      f"got head_dim {d}, block {block}")
        return _sparse_attention_rows(q, k, v, kv_num, kv_idx, block, scale, out)
    lse = torch.empty(B, Hq, n, device=q.device, dtype=torch.float32) if return_lse else None
    dt = _lib.dtype_code(q.dtype)
    ws_bytes = int(_lib.query("ssa_sparse_attn_workspace_size", dt, B, Hkv, n, d, block))
    flags = 0
    if prepared is not None:
        if vt is not None:
            raise ValueError("sparse_attention: pass vt or prepared, not both")
        if (prepared.shape != (B, Hkv, n, d) or prepared.dtype != v.dtype
                or prepared.block != block or prepared.device != q.device or dt == _lib.F32):
            raise ValueError("sparse_attention: `prepared` was built for other k / v / block")
        if prepared.used:
            raise ValueError("sparse_attention: a PreparedKV serves one call")
        prepared.used = True
        # (built on another stream, perhaps: keep its memory until this stream's work is done)
        prepared.ws.record_stream(torch.cuda.current_stream(q.device))
        ws, flags = prepared.ws, _lib.ATTN_PREPARED
    elif vt is not None and dt != _lib.F32:
        n_pad = -(-n // block) * block
        room = vt.untyped_storage().nbytes() - vt.storage_offset() * vt.element_size()
        if (tuple(vt.shape) != (B, Hkv, d, n_pad) or vt.dtype != v.dtype or room < ws_bytes
                or not vt.is_contiguous()):
            raise ValueError(f"vt {tuple(vt.shape)} {vt.dtype} is not the V^T workspace of this v "
                             f"(expected {(B, Hkv, d, n_pad)} {v.dtype} from transpose_v(v, {block}))")
        ws, flags = vt, _lib.ATTN_VT_READY
    else:
        ws = torch.empty(max(ws_bytes, 16), device=q.device, dtype=torch.uint8)
    if rotate and not torch.are_deterministic_algorithms_enabled():
        flags |= _lib.ATTN_ROTATE
    if exact:
        flags |= _lib.ATTN_EXACT
    strides = _lib.i64_array([*_bhn_strides(q), *_bhn_strides(k), *_bhn_strides(v),
                              *_bhn_strides(out)])
    _lib.call("ssa_sparse_attn_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dt,
              B, Hq, Hkv, n, d, block, strides, kv_num.data_ptr(), kv_idx.data_ptr(),
              kv_idx.shape[-1], float(scale), _lib.ptr(lse), flags, ws.data_ptr(), ws_bytes,
              _lib.stream_of(q))
    return (out, lse) if return_lse else out


# head dims the tiled prefill kernels serve (with block 64 or a multiple of 128): the MFMA
# kernel (bf16 / fp16) and the fp32 kernel; other head dims and blocks take the per-row kernel
TILED_HEAD_DIMS = (64, 128, 256, 512)
TILED_HEAD_DIMS_F32 = (64,)
_ROWS_WORKSPACE_LIMIT = 1 << 28


def _sparse_attention_rows(q, k, v, kv_num, kv_idx, block, scale, out):
    """The block-sparse prefill for head dims the tiled kernel does not serve: every query row of
    query block i takes block i's list, and the per-row kernel (ssa_decode_attend) attends the
    keys j <= t, j < n of those blocks -- the same mask_mod (kv <= q) & (kv < n). Query blocks
    are processed in chunks so that the per-row partials stay within _ROWS_WORKSPACE_LIMIT."""
    from .ivf_decode import attend_rows
    B, Hq, n, d = q.shape
    nb, W = kv_num.shape[-1], kv_idx.shape[-1]
    per_row = B * Hq * W * (d + 2) * 4
    chunk = max(1, _ROWS_WORKSPACE_LIMIT // (per_row * block))
    for i0 in range(0, nb, chunk):
        i1 = min(nb, i0 + chunk)
        r0, r1 = i0 * block, min(n, i1 * block)
        num = kv_num[:, :, i0:i1].repeat_interleave(block, dim=2)[:, :, :r1 - r0]
        idx = kv_idx[:, :, i0:i1].repeat_interleave(block, dim=2)[:, :, :r1 - r0]
        attend_rows(q[:, :, r0:r1], k, v, num, idx, r0, block, scale=scale,
                    out=out[:, :, r0:r1])
    return out


# ---------------------------------------------------------------------------------------------
# the reference's operator API
# ---------------------------------------------------------------------------------------------

def _finish(kv_num, kv_idx, nb, compact):
    if compact:
        return kv_num, kv_idx, None
    full, sel = expand_selection(kv_num, kv_idx, nb)
    return kv_num, full, sel


def block_route(q, k, block=BLOCK, top_c=8, local=1, routing="cumulant", compact=False):
    """Per query-block, the top-`top_c` causal key blocks (own block included in the competition)
    by <q̄,μ> + ½<q̄²,σ²_unbiased> (or <q̄,μ> unless routing == "cumulant"), OR the own block and
    `local` predecessors. Returns (kv_num (B,H,nb) int32, kv_idx (B,H,nb,nb) int32, sel bool).
    Reference: ssa/ssa_kernel.py:37-58."""
    B, H, n, d = q.shape
    if n % block:
        raise RuntimeError(f"block_route: n={n} is not a multiple of block={block}")
    nb = n // block
    qbar = block_summary(q, block, "qmean")
    cumulant = routing == "cumulant"
    mu, var, _ = block_summary(k, block, "unbiased" if cumulant else "pop")
    kv_num, kv_idx = route(qbar, mu, var if cumulant else None, None, "flat", int(top_c), 0.0,
                           int(local), 0.5 if cumulant else 0.0)
    return _finish(kv_num, kv_idx, nb, compact)


def block_route_budget(q, k, block=BLOCK, budget_frac=0.25, top_c=None, local=1, beta=2.0,
                       edgeworth=False, n_real=None, sub=None, proj=None, compact=False):
    """Budget router with gemma_ssa's semantics: per query block i keep the top
    ceil(budget_frac·i) (or `top_c`) strictly-past key blocks by <q̄,μ> + ½β<q̄²,σ²>
    (+ β²/6<q̄³,m3> if edgeworth), always OR the own block + `local` predecessors.
    `n_real` excludes pad keys from the block statistics. `sub` scores sub-blocks of that size and
    max-pools them to the block; `proj` (a (d, d') matrix, or an object with W_q / W_k) routes
    by the centroid score of the projected q̄ and μ. Returns (kv_num, kv_idx, sel).
    Reference: ssa/ssa_kernel.py:61-119."""
    B, H, n, d = q.shape
    if n % block:
        raise RuntimeError(f"block_route_budget: n={n} is not a multiple of block={block}")
    nb = n // block
    sub_sz = block if sub is None else int(sub)
    if sub_sz <= 0 or block % sub_sz:
        raise RuntimeError(f"block_route_budget: sub={sub} does not divide block={block}")
    pool = block // sub_sz  # sub-blocks per block, max-pooled (ssa/ssa_kernel.py:74-78,100)
    qbar = block_summary(q, block, "qmean")
    mu, var, m3 = block_summary(k, sub_sz, "pop", n_real=n_real,
                                with_m3=edgeworth and proj is None)
    if proj is not None:  # centroid score in the projected space (ssa/ssa_kernel.py:92-94)
        wq, wk = (proj.W_q, proj.W_k) if hasattr(proj, "W_q") else (proj, proj)
        kv_num, kv_idx = route(project_rows(qbar, wq), project_rows(mu, wk), None, None, "budget",
                               top_c, float(budget_frac), int(local), 0.0, pool=pool)
    else:
        kv_num, kv_idx = route(qbar, mu, var, m3, "budget", top_c, float(budget_frac), int(local),
                               0.5 * beta, beta ** 2 / 6.0, pool=pool)
    return _finish(kv_num, kv_idx, nb, compact)


def ssa_flex(q, k, v, block=BLOCK, top_c=8, local=1, routing="cumulant"):
    """Full SSA prefill: route (block_route) -> block-sparse causal attention, scale 1/√d.
    Reference: ssa/ssa_kernel.py:122-126."""
    kv_num, kv_idx, _ = block_route(q, k, block, top_c, local, routing, compact=True)
    return sparse_attention(q, k, v, kv_num, kv_idx, block)


def dense(q, k, v):
    """Dense causal attention baseline (torch SDPA), as ssa/ssa_kernel.py:129-130."""
    return F.scaled_dot_product_attention(q, k, v, is_causal=True)
