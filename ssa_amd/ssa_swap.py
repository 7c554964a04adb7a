"""Trainable SSA attention for the attention swap (drop-in for ssa/ssa_swap.py:32-63).

ssa_masked(q, k, v, block, top_c, local) keeps the reference's semantics -- every query routes on
its own: the cumulant score <q, mu_c> + 1/2 <q*q, var_c> against the statistics of the key blocks
(zero-padded to a block multiple, unbiased variance, the query's own block included with its later
keys), the top_c blocks that have begun at the query plus its own block and `local` predecessors,
then token-causal softmax attention over those keys -- and is differentiable in q, k and v (the
selection itself is not, as in the reference). On the GPU it runs the HIP router
(SSA_ROUTE_STARTED) and the per-row block-sparse attention forward/backward of libssa_hip.so;
there is no CPU path.

The module-level _SSA / _patched_sdpa / install / uninstall mirror the reference's swap switch:
with _SSA["on"], torch's scaled_dot_product_attention is replaced by ssa_masked.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib
from .ssa_kernel import block_summary, route

_SSA = {"on": False, "block": 64, "top_c": 4, "local": 2}
_orig_sdpa = F.scaled_dot_product_attention


def _strides(*ts):
    out = []
    for t in ts:
        out += [t.stride(0), t.stride(1), t.stride(2)]
    return _lib.i64_array(out)


def route_masked(q: torch.Tensor, k: torch.Tensor, block: int, top_c: int, local: int):
    """Per-query selection of ssa_masked (ssa/ssa_swap.py:40-51) -> compact (kv_num, kv_idx)
    (B, H, n) / (B, H, n, W): statistics of the zero-padded key blocks (unbiased variance),
    candidates = blocks begun at the query, top_c by score (ties: lowest block), own block and
    `local` predecessors."""
    n = q.shape[2]
    nb = -(-n // block)
    # the reference zero-pads k to nb * block rows and counts the zero rows in the statistics
    mu, var, _ = block_summary(k, block, "unbiased", n_real=nb * block)
    return route(q, mu, var, None, "started", int(top_c), 0.0, int(local), 0.5, query_pos=0,
                 block=block)


class _MaskedAttention(torch.autograd.Function):
    """Forward / backward over fixed per-row block lists (the selection is not differentiated)."""

    @staticmethod
    def forward(ctx, q, k, v, kv_num, kv_idx, block, scale):
        B, Hq, n, d = q.shape
        Hkv = k.shape[1]
        W = kv_idx.shape[-1]
        out = torch.empty(B, Hq, n, d, device=q.device, dtype=q.dtype)
        lse = torch.empty(B, Hq, n, device=q.device, dtype=torch.float32)
        wsb = int(_lib.query("ssa_masked_attn_workspace_size", B, Hq, n, W, d, int(block)))
        ws = torch.empty(wsb, device=q.device, dtype=torch.uint8)
        _lib.call("ssa_masked_attn_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                  lse.data_ptr(), _lib.dtype_code(q.dtype), B, Hq, Hkv, n, d, int(block),
                  _strides(q, k, v, out), kv_num.data_ptr(), kv_idx.data_ptr(), W, float(scale),
                  ws.data_ptr(), wsb, _lib.stream_of(q))
        ctx.save_for_backward(q, k, v, out, lse, kv_num, kv_idx)
        ctx.block, ctx.scale = int(block), float(scale)
        ctx.ws = ws  # its row masks serve the backward too
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, kv_num, kv_idx = ctx.saved_tensors
        B, Hq, n, d = q.shape
        Hkv = k.shape[1]
        W = kv_idx.shape[-1]
        dout = dout.to(out.dtype).contiguous()  # described by out's (contiguous) strides
        wsb = int(_lib.query("ssa_masked_attn_workspace_size", B, Hq, n, W, d, ctx.block))
        ws = ctx.ws  # the forward's workspace: its row masks are reused
        dt = _lib.dtype_code(q.dtype)
        strides = _strides(q, k, v, out)

        def run(gdt):
            dq = torch.empty(B, Hq, n, d, device=q.device, dtype=gdt)
            dk = torch.empty(B, Hkv, n, d, device=q.device, dtype=gdt)
            dv = torch.empty_like(dk)
            _lib.call("ssa_masked_attn_bwd", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                      out.data_ptr(), dout.data_ptr(), lse.data_ptr(), dq.data_ptr(),
                      dk.data_ptr(), dv.data_ptr(), dt, _lib.dtype_code(gdt),
                      _lib.MASKED_MASKS_READY, B, Hq, Hkv, n, d,
                      ctx.block, strides, kv_num.data_ptr(), kv_idx.data_ptr(), W, ctx.scale,
                      ws.data_ptr(), wsb, _lib.stream_of(q))
            return dq, dk, dv

        try:  # gradients written in the input type by the tiled kernels
            dq, dk, dv = run(q.dtype)
        except _lib.SSAError as e:
            if e.status != _lib.SSA_ERR_UNSUPPORTED or q.dtype == torch.float32:
                raise
            dq, dk, dv = run(torch.float32)  # per-row kernels: fp32 accumulation
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None, None


def ssa_masked(q, k, v, block, top_c, local):
    """Differentiable block-sparse SSA (ssa/ssa_swap.py:32-56): per query, a local window plus the
    top_c key blocks by cumulant score, token-causal, scale d**-0.5. q (B, Hq, n, d), k, v
    (B, Hkv, n, d) on the GPU; gradients flow to q, k and v through the attended keys."""
    _lib.require_device(q, k, v)
    if q.shape[1] % k.shape[1]:
        raise ValueError("ssa_masked: query heads must be a multiple of key heads")
    q, k, v = (t if t.stride(-1) == 1 and t.data_ptr() % 16 == 0 else t.contiguous()
               for t in (q, k, v))
    with torch.no_grad():
        kv_num, kv_idx = route_masked(q.detach(), k.detach(), block, top_c, local)
    return _MaskedAttention.apply(q, k, v, kv_num, kv_idx, int(block), q.shape[-1] ** -0.5)


def _patched_sdpa(q, k, v, *a, **kw):
    if _SSA["on"]:
        return ssa_masked(q, k, v, _SSA["block"], _SSA["top_c"], _SSA["local"])
    return _orig_sdpa(q, k, v, *a, **kw)


def install():
    """Route torch's scaled_dot_product_attention through ssa_masked while _SSA["on"]
    (the reference does F.scaled_dot_product_attention = _patched_sdpa in main())."""
    F.scaled_dot_product_attention = _patched_sdpa


def uninstall():
    F.scaled_dot_product_attention = _orig_sdpa


__all__ = ["ssa_masked", "route_masked", "_SSA", "_patched_sdpa", "install", "uninstall"]
