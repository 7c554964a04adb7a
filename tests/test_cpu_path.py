"""The torch-CPU restatement of the reference's path (oracle/cpu_path.py, bench.py's CPU
baseline) against the reference's own fixtures and the float64 oracle."""
import numpy as np
import torch

from oracle import cpu_path as C
from oracle import ssa_oracle as O
from ssa_amd import workloads as WL
from tests import golden_util as GU


def _compact(kv_num, kv_idx):
    kn = kv_num.numpy()
    W = int(kn.max())
    ki = kv_idx[..., :W].numpy()
    return kn, np.where(np.arange(W) < kn[..., None], ki, 0)


def test_cpu_route_budget_equals_reference_fixtures():
    """Same operator sequence as ssa/ssa_kernel.py:61-119 in float32: the C1 and C2 selections
    equal the reference's, row for row."""
    for name, cfg_name, kw in (("c1_budget", "C1", dict(top_c=8, local=1, beta=2.0)),
                               ("c1_frac", "C1", dict(budget_frac=0.25, local=1, beta=2.0)),
                               ("c2_budget", "C2", dict(top_c=32, local=2, beta=2.0))):
        p = WL.make(cfg_name)
        cfg = p["cfg"]
        g = GU.load(name)
        kv_num, kv_idx, sel = C.route_budget(torch.from_numpy(p["q"]), torch.from_numpy(p["k"]),
                                             cfg.block, **kw)
        kn, ki = _compact(kv_num, kv_idx)
        n, n_eq, _, bad = GU.compare_selections(kn, ki, g["kv_num"], g["kv_idx"])
        assert n_eq == n, (name, bad[:3])
        assert int(sel.sum()) == int(kv_num.sum())


def test_cpu_attention_matches_oracle():
    p = WL.make("C2", n=4096)
    cfg = p["cfg"]
    kv_num, kv_idx = O.route_budget(p["q"], p["k"], cfg.block, top_c=cfg.top_c, local=cfg.local,
                                    beta=cfg.beta)
    pairs = [(0, 0), (3, 17), (13, 63), (7, 40)]
    got = C.attend_blocks(torch.from_numpy(p["q"]), torch.from_numpy(p["k"]),
                          torch.from_numpy(p["v"]), torch.from_numpy(kv_num),
                          torch.from_numpy(kv_idx), cfg.block, pairs)
    ref = O.sparse_attention(p["q"], p["k"], p["v"], kv_num, kv_idx, cfg.block,
                             qblocks=sorted({i for _, i in pairs}), heads=sorted({h for h, _ in pairs}))
    for (h, i), o in got.items():
        sl = slice(i * cfg.block, (i + 1) * cfg.block)
        assert np.abs(o.numpy() - ref[0, h, sl]).max() < 1e-5, (h, i)


def test_cpu_decode_step_matches_reference_router_and_oracle():
    """decode_step over resident summaries: selections equal the reference's _selection_mask
    fixture at q_len = 1 (65,536-token C4-shaped cache), outputs the oracle's decode_attend."""
    g = GU.load("c4_query")
    p = WL.make("C4", n=65536 + 128)
    cfg = p["cfg"]
    k = torch.from_numpy(p["k"])
    v = torch.from_numpy(p["v"])
    for a, pos in enumerate(g["positions"].tolist()):
        ncomp = (pos + 1) // cfg.block
        kb = k[0, :, :ncomp * cfg.block].reshape(cfg.Hkv, ncomp, cfg.block, cfg.d)
        mu, var = kb.mean(2), kb.var(2, unbiased=False)
        out, lists = C.decode_step(torch.from_numpy(p["q"][0, :, pos]), k[0], v[0], mu, var, pos,
                                   cfg.block, cfg.top_c, cfg.local, cfg.beta)
        kn = np.array([[len(x) for x in lists]])
        ki = np.zeros((1, cfg.Hq, kn.max()), dtype=np.int64)
        for h, x in enumerate(lists):
            ki[0, h, :len(x)] = x
        n, n_eq, _, bad = GU.compare_selections(kn, ki, g["kv_num"][a][None], g["kv_idx"][a][None])
        assert n_eq == n, (pos, bad)
        G = cfg.Hq // cfg.Hkv
        for h in (0, 9):
            ref = O.decode_attend(p["q"][0, h, pos], p["k"][0, h // G], p["v"][0, h // G],
                                  lists[h], pos, cfg.block)
            assert np.abs(out[h].float().numpy() - ref).max() < 1e-5, (pos, h)
