"""Drop-in for the reference's transformers attention-interface boundary (ssa/gemma_ssa.py).

    SSAConfig, CFG, install_ssa(model, **cfg)            ssa/gemma_ssa.py:31-55,244-279
    ssa_attention_forward(module, query, key, value,
                          attention_mask, scaling, dropout, **kw)   ssa/gemma_ssa.py:183-241
    repeat_kv(x, n)                                      ssa/gemma_ssa.py:58-63

Dispatch mirrors the reference:
  * sliding layers (route_full_only) defer to the model's prior attention function;
  * prefill-shaped calls (q_len == kv_len > block) with impl "flex" (or "hip") take the fused
    path: query-block routing with block_route_budget semantics and n_real padding
    (ssa/gemma_ssa.py:140-180), then the block-sparse kernel, with donor/consumer sharing of the
    selection across layers (ssa/gemma_ssa.py:210-223);
  * everything else (decode q_len = 1, chunked prefill, impl "analytic") takes the per-query
    path of ssa/gemma_ssa.py:225-241: each query is routed over the key blocks complete at its
    position and attends its selected blocks, causally.
Both paths run on HIP kernels with GQA by index (no repeat_kv copies) and write the
(b, n, hq, d) output directly. Routing statistics are computed in fp32 (the reference's analytic
path computes them in the input dtype; parity is defined against its fp32 run).
Unlike the reference there is no CPU path: CPU tensors raise.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, fields
from types import SimpleNamespace

import torch

from . import _lib
from .ivf_decode import attend_rows
from .ssa_kernel import block_summary, project_rows, route, sparse_attention


@dataclass
class SSAConfig:
    block: int = 256
    budget_frac: float = 0.25
    top_c: int | None = None
    local_w: int = 1
    beta: float = 2.0
    route_full_only: bool = True
    edgeworth: bool = False
    dense_layers: tuple = ()
    impl: str = "analytic"
    share_route_from: int | None = None
    share_below: str = "per_layer"
    proj_path: str | None = None


CFG = SSAConfig()
_FALLBACK = None
_PROJ = None
_SHARE = {"sig": None, "bm": None}
ROUTE_MS = 0.0
# When True, route time is accumulated into ROUTE_MS (costs two device synchronisations per
# routed call, like the reference's timing at ssa/gemma_ssa.py:151-165).
TIME_ROUTE = False
# Per-layer key-block summaries of the per-query (decode) path, kept resident between calls:
# layer -> {"sig", "kv_len", "nc" (complete blocks summarised), "mu", "var", "m3" (capacity
# blocks)}. A call that continues the previous one (kv_len = previous kv_len + q_len, queries
# starting at the previous kv_len) summarises only the blocks it completes.
_DECODE = {}


def reset_decode_state():
    """Forgets the resident decode summaries of every layer. Needed only when a cache is edited
    in place at unchanged lengths (e.g. beam search reordering its batch): prefills, shorter or
    cropped caches and shape changes are detected and reset a layer's summaries by themselves."""
    _DECODE.clear()


def repeat_kv(x: torch.Tensor, n: int) -> torch.Tensor:
    """(b, h, s, d) -> (b, h*n, s, d), each head repeated n times (ssa/gemma_ssa.py:58-63)."""
    if n == 1:
        return x
    b, h, s, d = x.shape
    return x[:, :, None, :, :].expand(b, h, n, s, d).reshape(b, h * n, s, d)


NEG = float("-inf")  # additive mask value of a dropped key, as the reference's NEG


def _router_rows(x):
    """Query rows as the router reads them: 16-bit types as they are (their fp32 values are
    exact), anything else as fp32."""
    return x if x.dtype in (torch.float16, torch.bfloat16) else x.float()


def _block_stats(k: torch.Tensor, block: int):
    """Per-block mean / population variance / third central moment of the keys over the rows that
    exist (ssa/gemma_ssa.py:65-82): k (b, h, n, d) -> mu, var, m3 (b, h, nb, d) fp32 and nb."""
    n = k.shape[2]
    mu, var, m3 = block_summary(k, block, "pop", n_real=n, with_m3=True)
    return mu, var.clamp(min=0.0), m3, mu.shape[2]


def _selection_mask(q, k, cfg: SSAConfig, qpos=None, kpos=None):
    """Additive (0 / NEG) mask (b, hq, q_len, kv_len) of the per-query router
    (ssa/gemma_ssa.py:85-137): the top-budget blocks among those complete at each query's
    position, its own block and cfg.local_w predecessors, token-causal. Routing runs on the HIP
    router (SSA_ROUTE_QUERY); the dense mask is assembled on the device from its lists.
    `qpos` must be consecutive positions (the reference's default is the last q_len of a
    left-aligned sequence); `kpos` defaults to 0..kv_len-1."""
    _lib.require_device(q, k)
    b, hq, q_len, d = q.shape
    kv_len = k.shape[2]
    if qpos is None:
        pos0 = kv_len - q_len
    else:
        qp = torch.as_tensor(qpos).detach().to("cpu", torch.int64).view(-1)
        pos0 = int(qp[0])
        if qp.numel() != q_len or not torch.equal(qp, torch.arange(pos0, pos0 + q_len)):
            raise NotImplementedError("ssa_amd needs consecutive query positions")
    kpos_t = (torch.arange(kv_len, device=q.device) if kpos is None
              else torch.as_tensor(kpos, device=q.device).long())
    mu, var, m3 = block_summary(k, cfg.block, "pop", n_real=kv_len, with_m3=cfg.edgeworth)
    nb = mu.shape[2]
    kv_num, kv_idx = route(_router_rows(q), mu, var, m3 if cfg.edgeworth else None, "query",
                           cfg.top_c, cfg.budget_frac, cfg.local_w, 0.5 * cfg.beta,
                           cfg.beta ** 2 / 6.0 if cfg.edgeworth else 0.0, query_pos=pos0,
                           block=cfg.block)
    W = kv_idx.shape[-1]
    valid = torch.arange(W, device=q.device) < kv_num[..., None].long()
    sel = torch.zeros(b, hq, q_len, nb + 1, dtype=torch.bool, device=q.device)
    sel.scatter_(-1, torch.where(valid, kv_idx.long(), nb), True)
    key_sel = sel[..., :nb][..., kpos_t // cfg.block]
    qpos_t = torch.arange(pos0, pos0 + q_len, device=q.device)
    allow = key_sel & (qpos_t[:, None] >= kpos_t[None, :])[None, None]
    return torch.where(allow, 0.0, torch.tensor(NEG, device=q.device))


def load_projection(path, device="cuda"):
    """A trained routing projection saved as {"W_q": (d, d'), "W_k": (d, d'), "meta": {...}} by the
    reference's RoutingProjection.save (ssa/routing_space.py:43-51), loaded with weights_only=True
    (nothing in the file is executed). Returns an object with W_q / W_k (fp32, on `device`)."""
    d = torch.load(path, map_location=device, weights_only=True)
    return SimpleNamespace(W_q=d["W_q"].to(device).float(), W_k=d["W_k"].to(device).float(),
                           meta=d.get("meta", {}))


def _block_lists(query, key, cfg, dense, n):
    """Query-block routing of a prefill (block_route_budget semantics with n_real = n; with a
    loaded projection, the centroid score of the projected q̄ and μ, ssa/gemma_ssa.py:153-157)."""
    global ROUTE_MS
    blk = cfg.block
    if TIME_ROUTE:
        torch.cuda.synchronize()
        t0 = time.time()
    qbar = block_summary(query, blk, "qmean")
    proj = _PROJ
    mu, var, m3 = block_summary(key, blk, "pop", n_real=n,
                                with_m3=cfg.edgeworth and not dense and proj is None)
    if proj is not None:
        kv = route(project_rows(qbar, proj.W_q), project_rows(mu, proj.W_k), None, None, "budget",
                   None if dense else cfg.top_c, 1.0 if dense else cfg.budget_frac, cfg.local_w,
                   0.0)
    elif dense:
        kv = route(qbar, mu, var, None, "budget", None, 1.0, cfg.local_w, 0.5 * cfg.beta)
    else:
        kv = route(qbar, mu, var, m3, "budget", cfg.top_c, cfg.budget_frac, cfg.local_w,
                   0.5 * cfg.beta, cfg.beta ** 2 / 6.0)
    if TIME_ROUTE:
        torch.cuda.synchronize()
        ROUTE_MS += (time.time() - t0) * 1000
    return kv


def ssa_attention_forward(module, query, key, value, attention_mask=None, scaling=None,
                          dropout=0.0, **kwargs):
    """transformers attention-interface function. query (b, hq, n, d); key/value (b, hkv, n, d).
    Returns (attn_output (b, n, hq, d), None). `attention_mask` is ignored (causality comes from
    positions), as in the reference."""
    cfg = CFG
    is_sliding = bool(getattr(module, "is_sliding", False))
    if (cfg.route_full_only and is_sliding) and _FALLBACK is not None:
        return _FALLBACK(module, query, key, value, attention_mask,
                         scaling=scaling, dropout=dropout, **kwargs)
    _lib.require_device(query, key, value)
    if scaling is None:
        scaling = getattr(module, "scaling", 1.0)
    b, hq, q_len, d = query.shape
    kv_len = key.shape[2]
    nb_layer = (kv_len + cfg.block - 1) // cfg.block
    force_dense = getattr(module, "layer_idx", None) in cfg.dense_layers
    is_dense = force_dense or (cfg.top_c is not None and cfg.top_c >= nb_layer) \
        or (cfg.top_c is None and cfg.budget_frac >= 1.0)
    out = torch.empty(b, q_len, hq, d, device=query.device, dtype=query.dtype)

    if cfg.impl in ("flex", "hip") and q_len == kv_len and q_len > cfg.block:
        li = getattr(module, "layer_idx", None)
        # a prefill starts a sequence: the layer's resident decode summaries no longer apply
        _DECODE.pop(("layer", li) if li is not None else ("module", id(module)), None)
        donor = cfg.share_route_from
        lists = None
        if donor is not None and li is not None:
            if li < donor:
                is_dense = is_dense or cfg.share_below == "dense"
            elif li > donor:
                sig = (tuple(query.shape), kv_len, str(query.device))
                if _SHARE["sig"] == sig:
                    lists = _SHARE["bm"]
        if lists is None:
            lists = _block_lists(query, key, cfg, is_dense, q_len)
        if donor is not None and li == donor:
            _SHARE["sig"] = (tuple(query.shape), kv_len, str(query.device))
            _SHARE["bm"] = lists
        sparse_attention(query, key, value, lists[0], lists[1], cfg.block, scale=scaling,
                         out=out.transpose(1, 2))
        return out, None

    # per-query (analytic) path: query row r sits at absolute position pos0 + r
    cpos = kwargs.get("cache_position")
    if cpos is not None:
        cp = cpos.detach().to("cpu", torch.int64).view(-1)
        pos0 = int(cp[0])
        if cp.numel() != q_len or not torch.equal(cp, torch.arange(pos0, pos0 + q_len)):
            raise NotImplementedError("ssa_amd needs contiguous cache_position values")
    else:
        pos0 = kv_len - q_len
    if pos0 + q_len > kv_len or pos0 < 0:
        raise ValueError("query positions exceed the key length")
    # the edgeworth (third-cumulant) term joins the score as in ssa/gemma_ssa.py:101-102; a
    # dense call selects every causal block, so it needs no score terms beyond the first
    edge = cfg.edgeworth and not is_dense
    mu, var, m3 = _query_path_summaries(module, key, q_len, pos0, edge, cfg.block)
    rows = _router_rows(query)
    if is_dense:
        top_c, frac = nb_layer, 0.0
    else:
        top_c, frac = cfg.top_c, cfg.budget_frac
    kv_num, kv_idx = route(rows, mu, var, m3 if edge else None, "query", top_c, frac,
                           cfg.local_w, 0.5 * cfg.beta, cfg.beta ** 2 / 6.0 if edge else 0.0,
                           query_pos=pos0, block=cfg.block)
    attend_rows(query, key, value, kv_num, kv_idx, pos0, cfg.block, scale=scaling,
                out=out.transpose(1, 2))
    return out, None


def _query_path_summaries(module, key, q_len, pos0, with_m3, block):
    """mu, var, m3 (b, hkv, ceil(kv_len/block), d) fp32 for the per-query router. The router's
    candidates are the blocks complete at each query's position (ssa/gemma_ssa.py:109-110), all
    complete at kv_len, so only those entries are read: they are the population statistics of
    their rows (ssa/gemma_ssa.py:65-82), bit for bit the values block_summary gives over the
    whole key; the tail block's entry is not used. Decode steps continue the previous call, so a
    step summarises at most the one block it completes instead of the whole cache."""
    b, hkv, kv_len, d = key.shape
    nb = -(-kv_len // block)
    if torch.compiler.is_compiling():  # no Python-side state under tracing
        return block_summary(key, block, "pop", n_real=kv_len, with_m3=with_m3)
    li = getattr(module, "layer_idx", None)
    lk = ("layer", li) if li is not None else ("module", id(module))
    sig = (b, hkv, d, key.dtype, str(key.device), block, bool(with_m3))
    st = _DECODE.get(lk)
    if st is None or st["sig"] != sig or pos0 != st["kv_len"] or kv_len != st["kv_len"] + q_len:
        st = {"sig": sig, "kv_len": 0, "nc": 0, "mu": None, "var": None, "m3": None}
        _DECODE[lk] = st
    if st["mu"] is None or st["mu"].shape[2] < nb:  # capacity doubles, contents kept
        cap = max(nb, 2 * (0 if st["mu"] is None else st["mu"].shape[2]), 64)
        for name in ("mu", "var", "m3"):
            if name == "m3" and not with_m3:
                continue
            buf = torch.zeros(b, hkv, cap, d, device=key.device, dtype=torch.float32)
            if st[name] is not None:
                buf[:, :, :st["nc"]].copy_(st[name][:, :, :st["nc"]])
            st[name] = buf
    nc = kv_len // block
    if nc > st["nc"]:
        a = st["nc"]
        mu, var, m3 = block_summary(key[:, :, a * block:nc * block], block, "pop",
                                    with_m3=with_m3)
        st["mu"][:, :, a:nc].copy_(mu)
        st["var"][:, :, a:nc].copy_(var)
        if with_m3:
            st["m3"][:, :, a:nc].copy_(m3)
        st["nc"] = nc
    st["kv_len"] = kv_len
    return (st["mu"][:, :, :nb], st["var"][:, :, :nb],
            st["m3"][:, :, :nb] if with_m3 else None)


def install_ssa(model, **cfg_kwargs):
    """Registers ssa_attention_forward as the model's attention implementation, resetting every
    SSAConfig field not passed here to its default (ssa/gemma_ssa.py:244-279)."""
    global _FALLBACK, _PROJ
    defaults = SSAConfig()
    for f in fields(SSAConfig):
        setattr(CFG, f.name, getattr(defaults, f.name))
    for k, val in cfg_kwargs.items():
        setattr(CFG, k, val)
    _SHARE["sig"] = None
    _SHARE["bm"] = None
    _DECODE.clear()
    _PROJ = None
    if CFG.proj_path:
        _PROJ = load_projection(CFG.proj_path)
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    prior = getattr(model.config, "_attn_implementation", None) or "sdpa"
    if prior == "ssa":
        prior = None if _FALLBACK is not None else "sdpa"
    if prior is not None:
        try:
            _FALLBACK = ALL_ATTENTION_FUNCTIONS.get_interface(prior)
        except Exception:
            _FALLBACK = ALL_ATTENTION_FUNCTIONS.get("sdpa")
    ALL_ATTENTION_FUNCTIONS["ssa"] = ssa_attention_forward
    model.config._attn_implementation = "ssa"
    if hasattr(model.config, "get_text_config"):
        try:
            model.config.get_text_config()._attn_implementation = "ssa"
        except Exception:
            pass
    return model
