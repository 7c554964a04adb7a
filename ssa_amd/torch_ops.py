"""torch.library registrations of the HIP entry points (namespace `ssa_amd`), so that the drop-in
functions compose with torch.compile.

Under tracing (torch.compiler.is_compiling()) the public functions -- ssa_kernel.block_summary,
route, sparse_attention, ivf_decode.attend_rows and RoutedDecoder.step -- call these ops, which
the compiler keeps as opaque kernels; their fake implementations give the output shapes and
dtypes. Run eagerly, the public functions call the library directly and skip the dispatcher.

    ssa_amd::block_qmean(x, block) -> q_mean                      ssa/ssa_kernel.py:44,79
    ssa_amd::block_stats(x, block, unbiased, n_real, with_m3)     ssa/ssa_kernel.py:78-91,42-47
        -> (mu, var, m3)   (m3 has no elements unless with_m3)
    ssa_amd::route(rows, mu, var, m3, mode, top_c, budget_frac,   ssa/ssa_kernel.py:92-118,
                   local, coef2, coef3, query_pos, block, pool)   ssa/gemma_ssa.py:99-131
        -> (kv_num, kv_idx)   (top_c -1: budget_frac decides)
    ssa_amd::sparse_attention(q, k, v, kv_num, kv_idx, block, scale) -> out
    ssa_amd::sparse_attention_lse(...) -> (out, lse)              ssa/ssa_kernel.py:125-126
    ssa_amd::attend_rows(q, k, v, kv_num, kv_idx, pos, block, scale) -> out
                                                                  ssa/ivf_decode.py:49-62
    ssa_amd::decode_step(q, k_new, v_new, kcache!, vcache!, mu!, var!, kv_num!, kv_idx!,
                         workspace!, pos, block, top_c, budget_frac, local, coef2, scale) -> out
                                                                  ssa/ivf_decode.py:128-136
    (! = written in place; workspace None runs the allocation-free ssa_decode_step_static)
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _lib

_F32 = torch.float32


@torch.library.custom_op("ssa_amd::block_qmean", mutates_args=())
def block_qmean(x: Tensor, block: int) -> Tensor:
    from .ssa_kernel import _block_summary_impl
    return _block_summary_impl(x, block, "qmean", None, False)


@block_qmean.register_fake
def _(x, block):
    B, H, n, d = x.shape
    return x.new_empty(B, H, -(-n // block), d, dtype=_F32)


@torch.library.custom_op("ssa_amd::block_stats", mutates_args=())
def block_stats(x: Tensor, block: int, unbiased: bool, n_real: int,
                with_m3: bool) -> tuple[Tensor, Tensor, Tensor]:
    from .ssa_kernel import _block_summary_impl
    mu, var, m3 = _block_summary_impl(x, block, "unbiased" if unbiased else "pop",
                                      None if n_real < 0 else n_real, with_m3)
    return mu, var, (m3 if m3 is not None else mu.new_empty(0))


@block_stats.register_fake
def _(x, block, unbiased, n_real, with_m3):
    B, H, n, d = x.shape
    shape = (B, H, -(-n // block), d)
    return (x.new_empty(shape, dtype=_F32), x.new_empty(shape, dtype=_F32),
            x.new_empty(shape if with_m3 else (0,), dtype=_F32))


@torch.library.custom_op("ssa_amd::route", mutates_args=())
def route(rows: Tensor, mu: Tensor, var: Optional[Tensor], m3: Optional[Tensor], mode: str,
          top_c: int, budget_frac: float, local: int, coef2: float, coef3: float,
          query_pos: int, block: int, pool: int) -> tuple[Tensor, Tensor]:
    from .ssa_kernel import _route_impl
    return _route_impl(rows, mu, var, m3, mode, None if top_c < 0 else top_c, budget_frac, local,
                       coef2, coef3, query_pos, block, pool=pool)


@route.register_fake
def _(rows, mu, var, m3, mode, top_c, budget_frac, local, coef2, coef3, query_pos, block, pool):
    from .ssa_kernel import route_width
    B, Hq, nbq, _ = rows.shape
    nbk = mu.shape[2] // pool
    W = route_width(mode, nbq, nbk, None if top_c < 0 else top_c, budget_frac, local, query_pos,
                    block)
    return (rows.new_empty(B, Hq, nbq, dtype=torch.int32),
            rows.new_empty(B, Hq, nbq, W, dtype=torch.int32))


@torch.library.custom_op("ssa_amd::sparse_attention", mutates_args=())
def sparse_attention(q: Tensor, k: Tensor, v: Tensor, kv_num: Tensor, kv_idx: Tensor, block: int,
                     scale: float) -> Tensor:
    from .ssa_kernel import _sparse_attention_impl
    return _sparse_attention_impl(q, k, v, kv_num, kv_idx, block, scale)


@sparse_attention.register_fake
def _(q, k, v, kv_num, kv_idx, block, scale):
    return torch.empty_like(q, memory_format=torch.contiguous_format)


@torch.library.custom_op("ssa_amd::sparse_attention_lse", mutates_args=())
def sparse_attention_lse(q: Tensor, k: Tensor, v: Tensor, kv_num: Tensor, kv_idx: Tensor,
                         block: int, scale: float) -> tuple[Tensor, Tensor]:
    from .ssa_kernel import _sparse_attention_impl
    return _sparse_attention_impl(q, k, v, kv_num, kv_idx, block, scale, return_lse=True)


@sparse_attention_lse.register_fake
def _(q, k, v, kv_num, kv_idx, block, scale):
    B, Hq, n, _ = q.shape
    return (torch.empty_like(q, memory_format=torch.contiguous_format),
            q.new_empty(B, Hq, n, dtype=_F32))


@torch.library.custom_op("ssa_amd::attend_rows", mutates_args=())
def attend_rows(q: Tensor, k: Tensor, v: Tensor, kv_num: Tensor, kv_idx: Tensor, pos: int,
                block: int, scale: float) -> Tensor:
    from .ivf_decode import _attend_rows_impl
    return _attend_rows_impl(q, k, v, kv_num, kv_idx, pos, block, scale)


@attend_rows.register_fake
def _(q, k, v, kv_num, kv_idx, pos, block, scale):
    return torch.empty_like(q, memory_format=torch.contiguous_format)


@torch.library.custom_op("ssa_amd::decode_step",
                         mutates_args=("kcache", "vcache", "mu", "var", "kv_num", "kv_idx",
                                       "workspace"))
def decode_step(q: Tensor, k_new: Tensor, v_new: Tensor, kcache: Tensor, vcache: Tensor,
                mu: Tensor, var: Tensor, kv_num: Tensor, kv_idx: Tensor,
                workspace: Optional[Tensor], pos: int, block: int, top_c: int,
                budget_frac: float, local: int, coef2: float, scale: float) -> Tensor:
    B, Hq, d = q.shape
    Hkv, cap = kcache.shape[1], kcache.shape[2]
    out = torch.empty(B, Hq, d, device=q.device, dtype=kcache.dtype)
    strides = _lib.i64_array([q.stride(0), q.stride(1), k_new.stride(0), k_new.stride(1),
                              v_new.stride(0), v_new.stride(1), *kcache.stride()[:3],
                              *vcache.stride()[:3], out.stride(0), out.stride(1)])
    args = (q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), kcache.data_ptr(),
            vcache.data_ptr(), mu.data_ptr(), var.data_ptr(), out.data_ptr(),
            _lib.dtype_code(kcache.dtype), B, Hq, Hkv, cap, d, block, pos, strides, top_c,
            budget_frac, local, coef2, scale, kv_num.data_ptr(), kv_idx.data_ptr(),
            kv_idx.shape[-1])
    if workspace is None:
        _lib.call("ssa_decode_step_static", *args, _lib.stream_of(q))
    else:
        _lib.call("ssa_decode_step", *args, workspace.data_ptr(), workspace.numel(),
                  _lib.stream_of(q))
    return out


@decode_step.register_fake
def _(q, k_new, v_new, kcache, vcache, mu, var, kv_num, kv_idx, workspace, pos, block, top_c,
      budget_frac, local, coef2, scale):
    B, Hq, d = q.shape
    return q.new_empty(B, Hq, d, dtype=kcache.dtype)
