"""Writes the golden fixtures under tests/golden/ by running the REFERENCE implementation
(jonsmirl/ssa, read-only at /root/reference) on CPU in float32/float64.

Run once in the build container (the reference is not present on GPU boxes):

    python tests/golden/make_golden.py            # all cases
    python tests/golden/make_golden.py c1_budget  # selected cases

Each fixture is a small .npz of outputs only (selections as int16 compact lists, attention rows
as float32/float64) plus the sha256 of the inputs, which the tests regenerate from the same
seeded generators (ssa_amd.workloads / the seeds recorded here) and check against the hash.
Reference functions used (ssa/ssa_kernel.py, ssa/gemma_ssa.py, ssa/ssa_swap.py):
  block_route_budget :61-119, block_route :37-58, ssa_flex :122-126,
  _selection_mask :85-137 (also over the full 1M-token C4 cache),
  ssa_attention_forward :183-241 (impl="analytic", with and without edgeworth),
  ssa_masked :32-56 (forward and autograd backward).
"""
from __future__ import annotations

import hashlib
import sys
import time
from types import SimpleNamespace
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
REFERENCE = Path("/root/reference")

from ssa_amd import workloads as WL  # noqa: E402
from tests import golden_util as GU  # noqa: E402


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def reference():
    sys.path.insert(0, str(REFERENCE))
    from ssa import gemma_ssa, ssa_kernel  # noqa: E402
    return ssa_kernel, gemma_ssa


def compact_from_full(kv_num, kv_idx_full):
    """Reference (kv_num, argsort-order kv_idx) -> compact int16 (kv_num, kv_idx[..., :W])."""
    kv_num = kv_num.numpy().astype(np.int16)
    W = int(kv_num.max())
    ki = kv_idx_full[..., :W].numpy().astype(np.int16)
    # the compact contract pads with 0 beyond kv_num
    mask = np.arange(W)[None, None, None, :] < kv_num[..., None]
    return kv_num, np.where(mask, ki, 0).astype(np.int16)


def repeat_kv(x: torch.Tensor, n: int) -> torch.Tensor:
    b, h, s, d = x.shape
    return x[:, :, None].expand(b, h, n, s, d).reshape(b, h * n, s, d)


def route_case(name, cfg_name, variant="segmented", **kw):
    RK, _ = reference()
    p = WL.make(cfg_name, variant)
    cfg = p["cfg"]
    q = torch.from_numpy(p["q"])
    k = torch.from_numpy(p["k"])
    G = cfg.Hq // cfg.Hkv
    kk = repeat_kv(k, G) if G > 1 else k
    fn = kw.pop("fn", "budget")
    rk = dict(kw)
    if "proj_seed" in rk:      # one seeded (d, 16) projection used for queries and keys
        rk["proj"] = torch.from_numpy(WL.proj_matrix(rk.pop("proj_seed"), cfg.d))
    if "proj_pair_seed" in rk:  # an object with W_q / W_k (the trained-projection form)
        s0 = rk.pop("proj_pair_seed")
        rk["proj"] = SimpleNamespace(W_q=torch.from_numpy(WL.proj_matrix(s0, cfg.d)),
                                     W_k=torch.from_numpy(WL.proj_matrix(s0 + 1, cfg.d)))
    t0 = time.time()
    with torch.no_grad():
        if fn == "budget":
            kv_num, kv_idx, _ = RK.block_route_budget(q, kk, cfg.block, **rk)
        else:
            kv_num, kv_idx, _ = RK.block_route(q, kk, cfg.block, **rk)
    kn, ki = compact_from_full(kv_num, kv_idx)
    np.savez_compressed(HERE / f"{name}.npz", kv_num=kn, kv_idx=ki,
                        inputs_sha256=np.array(sha(p["q"], p["k"])),
                        meta=np.array(repr({"cfg": cfg_name, "variant": variant, "fn": fn, **kw})))
    print(f"{name}: rows={kn.size} W={ki.shape[-1]} ({time.time() - t0:.1f}s)")


def flex_case(name):
    """ssa_flex on C1 (fp32, CPU FlexAttention) -- the reference's own block-sparse output."""
    RK, _ = reference()
    p = WL.make("C1")
    q, k, v = (torch.from_numpy(p[x]) for x in ("q", "k", "v"))
    t0 = time.time()
    with torch.no_grad():
        out = RK.ssa_flex(q, k, v, block=64, top_c=8, local=1)
    np.savez_compressed(HERE / f"{name}.npz", out=out.numpy().astype(np.float32),
                        inputs_sha256=np.array(sha(p["q"], p["k"], p["v"])),
                        meta=np.array(repr({"cfg": "C1", "fn": "ssa_flex", "block": 64,
                                            "top_c": 8, "local": 1})))
    print(f"{name}: out {tuple(out.shape)} ({time.time() - t0:.1f}s)")


def query_case(name, n_cache=65536, positions=(65535, 65600, 65663)):
    """_selection_mask at q_len=1 (the exact per-query decode router) in float32 on a C4-shaped
    prefix: block set of each q-head for several decode positions."""
    _, RG = reference()
    p = WL.make("C4", n=n_cache + 128)
    cfg = p["cfg"]
    G = cfg.Hq // cfg.Hkv
    q = torch.from_numpy(p["q"])
    k = repeat_kv(torch.from_numpy(p["k"]), G)
    scfg = RG.SSAConfig(block=cfg.block, top_c=cfg.top_c, local_w=cfg.local, beta=cfg.beta)
    lists = []
    t0 = time.time()
    with torch.no_grad():
        for pos in positions:
            m = RG._selection_mask(q[:, :, pos:pos + 1], k[:, :, :pos + 1], scfg)  # (1,hq,1,pos+1)
            nb = -(-(pos + 1) // cfg.block)
            first = m[0, :, 0, ::cfg.block][:, :nb]                 # first key of each block
            lists.append([np.flatnonzero((first[h] == 0).numpy()).astype(np.int16)
                          for h in range(cfg.Hq)])
    W = max(len(x) for row in lists for x in row)
    kv_num = np.array([[len(x) for x in row] for row in lists], dtype=np.int16)
    kv_idx = np.zeros((len(positions), cfg.Hq, W), dtype=np.int16)
    for a, row in enumerate(lists):
        for h, x in enumerate(row):
            kv_idx[a, h, :len(x)] = x
    np.savez_compressed(HERE / f"{name}.npz", kv_num=kv_num, kv_idx=kv_idx,
                        positions=np.array(positions, dtype=np.int64),
                        inputs_sha256=np.array(sha(p["q"], p["k"])),
                        meta=np.array(repr({"cfg": "C4", "n_cache": n_cache,
                                            "fn": "_selection_mask", "top_c": cfg.top_c,
                                            "local_w": cfg.local})))
    print(f"{name}: positions={positions} W={W} ({time.time() - t0:.1f}s)")


def analytic_case(name, budget_frac=0.5, block=64, seed=11, skew=0.0, edgeworth=False):
    """ssa_attention_forward(impl='analytic') in float64: per-query routing + masked softmax,
    GQA 2:1, n not a multiple of the block; prefill and a q_len=1 decode row. With `edgeworth`
    the third-cumulant term joins the per-query score (ssa/gemma_ssa.py:101-102); `skew` gives
    the keys a skewed component so that the term changes selections."""
    _, RG = reference()
    from types import SimpleNamespace
    q, k, v = GU.analytic_inputs(seed, skew=skew)
    mod = SimpleNamespace(num_key_value_groups=q.shape[1] // k.shape[1], is_sliding=False,
                          scaling=0.125, layer_idx=0)
    RG.CFG = RG.SSAConfig(block=block, budget_frac=budget_frac, local_w=1, beta=2.0,
                          impl="analytic", edgeworth=edgeworth)
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    with torch.no_grad():
        full, _ = RG.ssa_attention_forward(mod, tq, tk, tv, scaling=0.125)
        inc, _ = RG.ssa_attention_forward(mod, tq[:, :, -1:], tk, tv, scaling=0.125)
    np.savez_compressed(HERE / f"{name}.npz", out=full.numpy(), out_last=inc.numpy(),
                        inputs_sha256=np.array(sha(q, k, v)),
                        meta=np.array(repr({"seed": seed, "skew": skew, "block": block,
                                            "budget_frac": budget_frac, "local_w": 1,
                                            "beta": 2.0, "scaling": 0.125,
                                            "edgeworth": edgeworth})))
    print(f"{name}: out {tuple(full.shape)}")


def query_1m_case(name, steps=GU.C4_1M_STEPS, ts=GU.C4_1M_TS):
    """_selection_mask at q_len=1 in float32 over the FULL C4 decode cache: the 1,048,576-token
    prefix of workloads.make_decode (the bench's decode workload) plus the appended tokens, at
    decode steps t (position n_cache + t; t = 127 completes a block)."""
    _, RG = reference()
    p = WL.make_decode(steps=steps)
    cfg = p["cfg"]
    n = p["n_cache"]
    G = cfg.Hq // cfg.Hkv
    q = torch.from_numpy(p["q"])
    k = torch.from_numpy(p["k"])
    scfg = RG.SSAConfig(block=cfg.block, top_c=cfg.top_c, local_w=cfg.local, beta=cfg.beta)
    lists = []
    t0 = time.time()
    with torch.no_grad():
        for t in ts:
            pos = n + t
            m = RG._selection_mask(q[:, :, t:t + 1], repeat_kv(k[:, :, :pos + 1], G), scfg)
            nb = -(-(pos + 1) // cfg.block)
            first = m[0, :, 0, ::cfg.block][:, :nb]
            lists.append([np.flatnonzero((first[h] == 0).numpy()).astype(np.int16)
                          for h in range(cfg.Hq)])
            del m
    W = max(len(x) for row in lists for x in row)
    kv_num = np.array([[len(x) for x in row] for row in lists], dtype=np.int16)
    kv_idx = np.zeros((len(ts), cfg.Hq, W), dtype=np.int16)
    for a, row in enumerate(lists):
        for h, x in enumerate(row):
            kv_idx[a, h, :len(x)] = x
    np.savez_compressed(HERE / f"{name}.npz", kv_num=kv_num, kv_idx=kv_idx,
                        steps=np.array(ts, dtype=np.int64),
                        positions=np.array([n + t for t in ts], dtype=np.int64),
                        inputs_sha256=np.array(sha(p["q"], p["k"])),
                        meta=np.array(repr({"cfg": "C4", "n_cache": n, "decode_steps": steps,
                                            "fn": "_selection_mask", "top_c": cfg.top_c,
                                            "local_w": cfg.local})))
    print(f"{name}: steps={ts} W={W} ({time.time() - t0:.1f}s)")


def c5_prefix_case(name):
    """block_route_budget at C5's geometry (fp16, block 256, top_c 64, local 1, beta 2) on a
    2,097,152-token prefix (8192 blocks) drawn by workloads.make_c5_prefix: causality makes each
    query block's selection independent of the tokens after it, so these rows are C5's rows on
    these inputs."""
    RK, _ = reference()
    p = WL.make_c5_prefix()
    cfg = p["cfg"]
    q, k = torch.from_numpy(p["q"]), torch.from_numpy(p["k"])
    t0 = time.time()
    with torch.no_grad():
        kv_num, kv_idx, _ = RK.block_route_budget(q.half(), k.half(), cfg.block, top_c=cfg.top_c,
                                                  local=cfg.local, beta=cfg.beta)
    kn, ki = compact_from_full(kv_num, kv_idx)
    np.savez_compressed(HERE / f"{name}.npz", kv_num=kn, kv_idx=ki,
                        inputs_sha256=np.array(sha(p["q"], p["k"])),
                        meta=np.array(repr({"cfg": "C5 prefix", "n": p["q"].shape[2],
                                            "dtype": "fp16", "block": cfg.block,
                                            "top_c": cfg.top_c, "local": cfg.local,
                                            "beta": cfg.beta})))
    print(f"{name}: rows={kn.size} W={ki.shape[-1]} ({time.time() - t0:.1f}s)")


def masked_case(name):
    """ssa_swap.ssa_masked in float32 on CPU: forward output and the gradients of sum(out * g)
    with respect to q, k and v (torch autograd through the reference's masked dense form)."""
    sys.path.insert(0, str(REFERENCE))
    from ssa import ssa_swap as RS  # noqa: E402
    seed, (b, h, n, d), block, top_c, local = GU.MASKED_CASES[name]
    q, k, v, g = GU.masked_inputs(seed, b, h, n, d)
    tq, tk, tv = (torch.from_numpy(x).requires_grad_(True) for x in (q, k, v))
    t0 = time.time()
    out = RS.ssa_masked(tq, tk, tv, block, top_c, local)
    out.backward(torch.from_numpy(g))
    np.savez_compressed(HERE / f"{name}.npz", out=out.detach().numpy(), dq=tq.grad.numpy(),
                        dk=tk.grad.numpy(), dv=tv.grad.numpy(),
                        inputs_sha256=np.array(sha(q, k, v, g)),
                        meta=np.array(repr({"seed": seed, "shape": (b, h, n, d), "block": block,
                                            "top_c": top_c, "local": local})))
    print(f"{name}: out {tuple(out.shape)} ({time.time() - t0:.1f}s)")


CASES = {
    "c1_budget": lambda: route_case("c1_budget", "C1", top_c=8, local=1, beta=2.0),
    "c1_frac": lambda: route_case("c1_frac", "C1", budget_frac=0.25, local=1, beta=2.0),
    "c1_flat": lambda: route_case("c1_flat", "C1", fn="flat", top_c=8, local=1),
    "c2_budget": lambda: route_case("c2_budget", "C2", top_c=32, local=2, beta=2.0),
    "c2_edgeworth": lambda: route_case("c2_edgeworth", "C2", top_c=32, local=2, beta=2.0,
                                       edgeworth=True),
    "c3_budget_seg": lambda: route_case("c3_budget_seg", "C3", "segmented", top_c=64, local=2,
                                        beta=2.0),
    "c3_budget_lit": lambda: route_case("c3_budget_lit", "C3", "literal", top_c=64, local=2,
                                        beta=2.0),
    "c1_sub16": lambda: route_case("c1_sub16", "C1", top_c=8, local=1, beta=2.0, sub=16),
    "c2_sub16": lambda: route_case("c2_sub16", "C2", top_c=32, local=2, beta=2.0, sub=16),
    "c1_proj": lambda: route_case("c1_proj", "C1", top_c=8, local=1, proj_seed=31),
    "c2_proj_pair": lambda: route_case("c2_proj_pair", "C2", top_c=32, local=2,
                                       proj_pair_seed=41),
    "c4_query": lambda: query_case("c4_query"),
    "c1_flex_out": lambda: flex_case("c1_flex_out"),
    "analytic_gqa": lambda: analytic_case("analytic_gqa"),
    "analytic_gqa_edgeworth": lambda: analytic_case("analytic_gqa_edgeworth", seed=12, skew=0.7,
                                                    edgeworth=True),
    "c4_query_1m": lambda: query_1m_case("c4_query_1m"),
    "c5_prefix": lambda: c5_prefix_case("c5_prefix"),
    "swap_masked_b16": lambda: masked_case("swap_masked_b16"),
    "swap_masked_b64": lambda: masked_case("swap_masked_b64"),
}

if __name__ == "__main__":
    torch.set_num_threads(8)
    names = sys.argv[1:] or list(CASES)
    for nm in names:
        CASES[nm]()
