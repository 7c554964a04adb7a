"""Drop-in for the reference's routed decode (ssa/ivf_decode.py) on gfx950 HIP kernels.

    decode_attend(qvec, k, v, blocks, pos, block)   ssa/ivf_decode.py:49-62
    dense_decode(qvec, k, v, pos)                   ssa/ivf_decode.py:65-74 (baseline arm)
    attend_rows(q, k, v, kv_num, kv_idx, pos, ...)  batched per-query form (many heads / rows)
    RoutedDecoder                                   the per-step loop of ssa/ivf_decode.py:112-136

The reference selects decode blocks with an approximate faiss IVF search over block means
(ssa/ivf_decode.py:88-93,120-125). RoutedDecoder instead routes each step with the exact
cumulant router of ssa/gemma_ssa.py:85-137 at q_len = 1 (keep top-`top_c` of the complete
blocks by <q,μ> + ½β<q²,σ²>, plus the own block and `local` predecessors), keeping μ/σ² of
every complete block resident and summarising the tail block in the step that completes it.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import _lib
from .ssa_kernel import BLOCK, _bhn_strides, block_summary, route_width


def attend_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_num: torch.Tensor,
                kv_idx: torch.Tensor, pos: int, block: int, scale: float | None = None,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-query sparse attention: q (B, Hq, nq, d); caches k, v (B, Hkv, cap, d); row r of
    head (b, h) sits at absolute position pos + r and attends keys <= pos + r of the blocks
    kv_idx[b, h, r, :kv_num[b, h, r]] (fp32 softmax, output in q's dtype)."""
    if torch.compiler.is_compiling():
        from . import torch_ops as T
        sc = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
        o = T.attend_rows(q, k, v, kv_num, kv_idx, int(pos), int(block), sc)
        if out is not None:
            out.copy_(o)
            o = out
        return o
    return _attend_rows_impl(q, k, v, kv_num, kv_idx, pos, block, scale, out)


def _attend_rows_impl(q, k, v, kv_num, kv_idx, pos, block, scale=None, out=None):
    _lib.require_device(q, k, v, kv_num, kv_idx)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share a dtype")
    B, Hq, nq, d = q.shape
    Hkv, cap = k.shape[1], k.shape[2]
    if out is None:
        out = torch.empty(B, Hq, nq, d, device=q.device, dtype=q.dtype)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    kv_num = kv_num.to(torch.int32).contiguous()
    kv_idx = kv_idx.to(torch.int32).contiguous()
    W = kv_idx.shape[-1]
    ws_bytes = int(_lib.query("ssa_decode_attend_workspace_size", B, Hq, nq, W, d))
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    strides = _lib.i64_array([*_bhn_strides(q), *_bhn_strides(k), *_bhn_strides(v),
                              *_bhn_strides(out)])
    _lib.call("ssa_decode_attend", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
              _lib.dtype_code(q.dtype), B, Hq, Hkv, nq, cap, d, block, int(pos), strides,
              kv_num.data_ptr(), kv_idx.data_ptr(), W, float(scale), ws.data_ptr(), ws_bytes,
              _lib.stream_of(q))
    return out


@torch.no_grad()
def decode_attend(qvec, k, v, blocks, pos, block=BLOCK):
    """One decode attention row over the selected blocks, clipped causally at `pos`, fp32 softmax
    with scale 1/√d; returns (d,) in qvec's dtype. Reference: ssa/ivf_decode.py:49-62."""
    ids = sorted(set(int(x) for x in blocks))
    d = qvec.shape[-1]
    dev = qvec.device
    if not ids:
        return torch.zeros(d, device=dev, dtype=qvec.dtype)
    kv_num = torch.tensor([[[len(ids)]]], device=dev, dtype=torch.int32)
    kv_idx = torch.tensor([[[ids]]], device=dev, dtype=torch.int32)
    out = attend_rows(qvec.reshape(1, 1, 1, d), k.view(1, 1, *k.shape), v.view(1, 1, *v.shape),
                      kv_num, kv_idx, int(pos), block)
    return out.view(d)


@torch.no_grad()
def dense_decode(qvec, k, v, pos):
    """Dense decode baseline: one SDPA row over the whole causal prefix [0..pos]
    (ssa/ivf_decode.py:65-74)."""
    d = qvec.shape[-1]
    out = F.scaled_dot_product_attention(qvec.view(1, 1, 1, d), k[:pos + 1].view(1, 1, pos + 1, d),
                                         v[:pos + 1].view(1, 1, pos + 1, d))
    return out.view(d)


@torch.no_grad()
def dense_decode_naive(qvec, k, v, pos):
    """The reference's earlier dense decode (ssa/ivf_decode.py:77-85): the prefix K/V [0..pos]
    upcast to fp32 every step, softmax(q.K^T / sqrt(d)) V in fp32, cast to qvec's dtype. Kept as
    the side-by-side check of dense_decode, as the reference keeps it."""
    d = qvec.shape[-1]
    kp, vp = k[:pos + 1].float(), v[:pos + 1].float()
    w = torch.softmax((qvec.float() @ kp.T) / math.sqrt(d), dim=-1)
    return (w @ vp).to(qvec.dtype)


class RoutedDecoder:
    """A KV cache with resident block summaries and the fused routed decode step.

    cache: (B, Hkv, capacity, d) in `dtype`; summaries μ, σ² (population) of every complete
    block in fp32. step(q, k_new, v_new) appends the token at the next position, summarises the
    block it completes, routes q over the complete blocks and attends -- one ssa_decode_step
    call, no host synchronisation.
    """

    def __init__(self, batch, hq, hkv, d, capacity, block=BLOCK, top_c=64, budget_frac=None,
                 local=1, beta=2.0, dtype=torch.bfloat16, device="cuda", scale=None,
                 static_scratch=False):
        if hq % hkv:
            raise ValueError("hq must be a multiple of hkv")
        if top_c is None and budget_frac is None:
            raise ValueError("give top_c or budget_frac")
        self.B, self.Hq, self.Hkv, self.d = batch, hq, hkv, d
        self.block = block
        self.capacity = -(-capacity // block) * block
        self.nbk = self.capacity // block
        self.top_c = -1 if top_c is None else int(top_c)
        self.budget_frac = 0.0 if budget_frac is None else float(budget_frac)
        self.local = int(local)
        self.coef2 = 0.5 * beta
        self.scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
        self.dtype = dtype
        dev = torch.device(device)
        self.W = route_width("query", 1, self.nbk, None if top_c is None else top_c,
                             self.budget_frac, self.local, self.capacity - 1, block)
        ws = int(_lib.query("ssa_decode_step_workspace_size", batch, hq, self.capacity, d, block,
                            self.W))
        # static_scratch: steps run ssa_decode_step_static, whose scratch is the library's own
        # device array (no workspace here; steps with step(out=...) allocate nothing)
        self.static_scratch = bool(static_scratch)
        if self.static_scratch and ws > _lib.DECODE_STATIC_SCRATCH_BYTES:
            raise ValueError(f"a step needs {ws} bytes of scratch, more than the library's static "
                             f"{_lib.DECODE_STATIC_SCRATCH_BYTES}")
        self.kcache = torch.zeros(batch, hkv, self.capacity, d, device=dev, dtype=dtype)
        self.vcache = torch.zeros_like(self.kcache)
        self.mu = torch.zeros(batch, hkv, self.nbk, d, device=dev, dtype=torch.float32)
        self.var = torch.zeros_like(self.mu)
        self.kv_num = torch.zeros(batch, hq, device=dev, dtype=torch.int32)
        self.kv_idx = torch.zeros(batch, hq, self.W, device=dev, dtype=torch.int32)
        self.workspace = None if self.static_scratch else torch.empty(ws, device=dev,
                                                                      dtype=torch.uint8)
        self.pos = 0

    @torch.no_grad()
    def prefill(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Loads a prefix k, v (B, Hkv, n, d) and summarises its complete blocks."""
        n = k.shape[2]
        if n > self.capacity:
            raise ValueError("prefix longer than the cache")
        self.kcache[:, :, :n].copy_(k)
        self.vcache[:, :, :n].copy_(v)
        nc = n // self.block
        if nc:
            mu, var, _ = block_summary(self.kcache[:, :, :nc * self.block], self.block, "pop")
            self.mu[:, :, :nc].copy_(mu)
            self.var[:, :, :nc].copy_(var)
        self.pos = n

    @torch.no_grad()
    def step(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
             out: torch.Tensor | None = None) -> torch.Tensor:
        """q (B, Hq, d), k_new/v_new (B, Hkv, d) -> attention output (B, Hq, d). The selection
        is left in self.kv_num (B, Hq) / self.kv_idx (B, Hq, W)."""
        _lib.require_device(q, k_new, v_new)
        if self.pos >= self.capacity:
            raise RuntimeError("KV cache is full")
        for name, t, shape in (("q", q, (self.B, self.Hq, self.d)),
                               ("k_new", k_new, (self.B, self.Hkv, self.d)),
                               ("v_new", v_new, (self.B, self.Hkv, self.d))):
            if t.dtype != self.dtype:
                raise TypeError(f"step: {name} is {t.dtype}, the cache holds {self.dtype}")
            if tuple(t.shape) != shape:
                raise ValueError(f"step: {name} has shape {tuple(t.shape)}, expected {shape}")
            if t.stride(-1) != 1:
                raise ValueError(f"step: {name} needs a contiguous last dimension")
        if torch.compiler.is_compiling():
            from . import torch_ops as T
            o = T.decode_step(q, k_new, v_new, self.kcache, self.vcache, self.mu, self.var,
                              self.kv_num, self.kv_idx, self.workspace, self.pos, self.block,
                              self.top_c, self.budget_frac, self.local, self.coef2, self.scale)
            self.pos += 1
            if out is not None:
                out.copy_(o)
                o = out
            return o
        if out is None:
            out = torch.empty(self.B, self.Hq, self.d, device=q.device, dtype=self.dtype)
        elif (out.dtype != self.dtype or tuple(out.shape) != (self.B, self.Hq, self.d)
              or out.stride(-1) != 1):
            raise ValueError(f"step: out must be a ({self.B}, {self.Hq}, {self.d}) {self.dtype} "
                             "tensor with a contiguous last dimension")
        kc, vc = self.kcache, self.vcache
        strides = _lib.i64_array([q.stride(0), q.stride(1), k_new.stride(0), k_new.stride(1),
                                  v_new.stride(0), v_new.stride(1), kc.stride(0), kc.stride(1),
                                  kc.stride(2), vc.stride(0), vc.stride(1), vc.stride(2),
                                  out.stride(0), out.stride(1)])
        args = (q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                self.mu.data_ptr(), self.var.data_ptr(), out.data_ptr(),
                _lib.dtype_code(self.dtype), self.B, self.Hq, self.Hkv, self.capacity, self.d,
                self.block, self.pos, strides, self.top_c, self.budget_frac, self.local,
                self.coef2, self.scale, self.kv_num.data_ptr(), self.kv_idx.data_ptr(), self.W)
        if self.static_scratch:
            _lib.call("ssa_decode_step_static", *args, _lib.stream_of(q))
        else:
            _lib.call("ssa_decode_step", *args, self.workspace.data_ptr(), self.workspace.numel(),
                      _lib.stream_of(q))
        self.pos += 1
        return out
