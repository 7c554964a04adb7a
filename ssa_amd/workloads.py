"""Seeded synthetic inputs for the five benchmark configurations (C1-C5).

Inputs are drawn with NumPy's PCG64 (`default_rng(seed)`), so they are bit-identical on every
host, then rounded once to the configuration's dtype with torch (round-to-nearest-even). Arrays
are (B, H, n, d) float32 holding values exactly representable in the target dtype.

  C1 (seed 0): 1 head, fp32, n=4096, d=64, block 64, top_c 8, local 1, beta 2; Q,K,V ~ N(0,1);
      16 needles: probe rows t_j in the last quarter, a key at a random earlier position
      (at least one block before the probe's block) set to 3.0 * q_t/|q_t|, its value one-hot e_j.
  C2 (seed 1): bf16, n=32768, 14q/2kv heads, block 64, top_c 32, local 2, beta 2;
      K,V ~ N(0,1) * s_h with s_h ~ U[0.5, 2]^64 per key head; Q ~ N(0,1); 64 needles per key
      head (key = 4 * q_probe/|q_probe| for a probe query of that group, >= 2 blocks earlier;
      value one-hot).
  C3 (seed 2): bf16, n=131072, 14q/2kv, block 128, top_c 64, local 2, beta 2; keys from a
      256-component Gaussian mixture (means N(0,1), within-component std 0.3). variant
      "segmented": the component is constant over runs of 32 tokens (blocks get non-trivial
      spread); "literal": the component is drawn per token. Q, V ~ N(0,1).
  C4 (seed 3): decode, bf16, 14q/2kv, cache 1,048,576 (+steps), block 128, top_c 64, local 1
      (the last two blocks), beta 2; K/V as C3 "segmented" with 8 needles per key head.
  C5 (seed 4): 1 head, fp16, n=12,582,912, block 256, top_c 64, local 1, beta 2; Q,K,V ~ N(0,1)
      with 1024 needles. Generated on the device (torch Philox, seeded) -- 2.4e9 samples are too
      slow for NumPy in a benchmark run; its parity tests use size-independent properties.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass
class Config:
    name: str
    B: int
    Hq: int
    Hkv: int
    n: int
    d: int
    block: int
    top_c: int
    local: int
    beta: float
    dtype: torch.dtype
    seed: int
    extra: dict = field(default_factory=dict)

    @property
    def nb(self) -> int:
        return -(-self.n // self.block)


C1 = Config("C1", 1, 1, 1, 4096, 64, 64, 8, 1, 2.0, torch.float32, 0)
C2 = Config("C2", 1, 14, 2, 32768, 64, 64, 32, 2, 2.0, torch.bfloat16, 1)
C3 = Config("C3", 1, 14, 2, 131072, 64, 128, 64, 2, 2.0, torch.bfloat16, 2)
C4 = Config("C4", 1, 14, 2, 1048576, 64, 128, 64, 1, 2.0, torch.bfloat16, 3)
C5 = Config("C5", 1, 1, 1, 12582912, 64, 256, 64, 1, 2.0, torch.float16, 4)
CONFIGS = {c.name: c for c in (C1, C2, C3, C4, C5)}


def round_to(x: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Rounds float32 values to `dtype` (RNE) and returns them as float32."""
    if dtype == torch.float32:
        return x.astype(np.float32, copy=False)
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dtype).float().numpy()


def _normal(rng, shape):
    return rng.standard_normal(shape, dtype=np.float32)


def _plant(q, k, v, rng, nneedle, margin, group, block, min_gap_blocks, probe_lo):
    """Plants needles: for a random probe query t (>= probe_lo) of a random query head of each
    key head, a key at a random position at least `min_gap_blocks` blocks before t's block is set
    to margin * q_t/|q_t| and its value row to a one-hot vector. Returns (kvh, qh, probe, pos)."""
    B, Hkv, n, d = k.shape
    rec = []
    for kvh in range(Hkv):
        for j in range(nneedle):
            qh = kvh * group + int(rng.integers(group))
            t = int(rng.integers(probe_lo, n))
            hi = (t // block - min_gap_blocks + 1) * block
            if hi <= 0:
                continue
            p = int(rng.integers(0, hi))
            qt = q[0, qh, t]
            k[0, kvh, p] = margin * qt / np.linalg.norm(qt)
            v[0, kvh, p] = 0.0
            v[0, kvh, p, j % d] = 1.0
            rec.append((kvh, qh, t, p))
    return np.array(rec, dtype=np.int64).reshape(-1, 4)


def _gmm_keys(rng, Hkv, n, d, ncomp=256, std=0.3, run=32, literal=False):
    means = _normal(rng, (Hkv, ncomp, d))
    nruns = n if literal else -(-n // run)
    comp = rng.integers(0, ncomp, size=(Hkv, nruns))
    if not literal:
        comp = np.repeat(comp, run, axis=1)[:, :n]
    k = np.empty((1, Hkv, n, d), dtype=np.float32)
    for h in range(Hkv):
        k[0, h] = means[h][comp[h]] + std * _normal(rng, (n, d))
    return k


def make(name: str, variant: str = "segmented", n: int | None = None):
    """Host inputs of configuration `name` (C1-C4): dict with q, k, v float32 arrays already
    rounded to the config dtype, the Config, and the planted needles. `n` overrides the sequence
    length: a smaller instance drawn the same way (not a prefix of the full-length draw), used for
    reduced parity cases."""
    cfg = CONFIGS[name]
    rng = np.random.default_rng(cfg.seed)
    N = cfg.n if n is None else n
    G = cfg.Hq // cfg.Hkv
    needles = np.zeros((0, 4), dtype=np.int64)
    if name == "C1":
        q = _normal(rng, (1, 1, N, cfg.d))
        k = _normal(rng, (1, 1, N, cfg.d))
        v = _normal(rng, (1, 1, N, cfg.d))
        needles = _plant(q, k, v, rng, 16, 3.0, 1, cfg.block, 2, 3 * N // 4)
    elif name == "C2":
        s = rng.uniform(0.5, 2.0, size=(cfg.Hkv, cfg.d)).astype(np.float32)
        q = _normal(rng, (1, cfg.Hq, N, cfg.d))
        k = _normal(rng, (1, cfg.Hkv, N, cfg.d)) * s[None, :, None, :]
        v = _normal(rng, (1, cfg.Hkv, N, cfg.d)) * s[None, :, None, :]
        needles = _plant(q, k, v, rng, 64, 4.0, G, cfg.block, 2, 2 * cfg.block)
    elif name in ("C3", "C4"):
        q = _normal(rng, (1, cfg.Hq, N, cfg.d))
        k = _gmm_keys(rng, cfg.Hkv, N, cfg.d, literal=(variant == "literal"))
        v = _normal(rng, (1, cfg.Hkv, N, cfg.d))
        if name == "C4":
            needles = _plant(q, k, v, rng, 8, 4.0, G, cfg.block, 2, 2 * cfg.block)
    else:
        raise ValueError(f"{name}: host generation covers C1-C4 (C5 uses make_c5_device)")
    q, k, v = (round_to(x, cfg.dtype) for x in (q, k, v))
    return {"cfg": cfg, "q": q, "k": k, "v": v, "needles": needles, "variant": variant}


def proj_matrix(seed: int, din: int = 64, dout: int = 16) -> np.ndarray:
    """Seeded routing projection (din, dout) float32 for block_route_budget(proj=...) cases:
    N(0,1) / sqrt(din) from default_rng(seed)."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((din, dout)) / np.sqrt(din)).astype(np.float32)


def to_device(x: np.ndarray, dtype: torch.dtype, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def make_c5_device(device="cuda", n: int | None = None):
    """C5 inputs generated on the device: q, k, v (1, 1, n, 64) fp16 ~ N(0,1) (torch Philox,
    seed 4) with 1024 needles (key = 3 * q_probe/|q_probe| at least two blocks before the
    probe's block, value one-hot)."""
    cfg = C5
    N = cfg.n if n is None else n
    g = torch.Generator(device=device).manual_seed(cfg.seed)
    out = []
    for _ in range(3):
        t = torch.empty(1, 1, N, cfg.d, device=device, dtype=cfg.dtype)
        t.view(-1).normal_(generator=g)
        out.append(t)
    q, k, v = out
    rng = np.random.default_rng(cfg.seed)
    probes = rng.integers(4 * cfg.block, N, size=1024)
    rec = []
    for j, t in enumerate(probes.tolist()):
        hi = (t // cfg.block - 1) * cfg.block
        p = int(rng.integers(0, hi))
        qt = q[0, 0, t].float()
        k[0, 0, p] = (3.0 * qt / qt.norm()).to(cfg.dtype)
        v[0, 0, p].zero_()
        v[0, 0, p, j % cfg.d] = 1.0
        rec.append((0, 0, t, p))
    return {"cfg": cfg, "q": q, "k": k, "v": v, "needles": np.array(rec, dtype=np.int64)}


def make_c5_prefix(n: int = 2_097_152, seed: int = 104, nneedle: int = 170):
    """C5's geometry (1 head, fp16, d 64, block 256) on a host-drawn prefix for the router's
    reference fixture: q, k, v (1, 1, n, 64) ~ N(0,1) from default_rng(seed), rounded to fp16,
    with `nneedle` needles (C5's density: 1024 per 12.6M tokens) planted as in make_c5_device
    (key = 3 * q_probe/|q_probe| at least one block before the probe's block, value one-hot)."""
    cfg = C5
    rng = np.random.default_rng(seed)
    q = _normal(rng, (1, 1, n, cfg.d))
    k = _normal(rng, (1, 1, n, cfg.d))
    v = _normal(rng, (1, 1, n, cfg.d))
    needles = _plant(q, k, v, rng, nneedle, 3.0, 1, cfg.block, 2, 4 * cfg.block)
    q, k, v = (round_to(x, cfg.dtype) for x in (q, k, v))
    return {"cfg": cfg, "q": q, "k": k, "v": v, "needles": needles}


def make_decode(n_cache: int | None = None, steps: int = 64):
    """C4 decode inputs: a KV prefix of n_cache tokens (K from the segmented Gaussian mixture,
    V ~ N(0,1), 8 needles per key head planted for the decode queries) plus `steps` tokens to
    append, and one query per step per query head. Drawn from default_rng(seed 3) in its own
    order (only the decoded queries are generated), so it is a different draw than make("C4")."""
    cfg = C4
    n = cfg.n if n_cache is None else n_cache
    total = n + steps
    rng = np.random.default_rng(cfg.seed)
    k = _gmm_keys(rng, cfg.Hkv, total, cfg.d)
    v = _normal(rng, (1, cfg.Hkv, total, cfg.d))
    q = _normal(rng, (1, cfg.Hq, steps, cfg.d))
    G = cfg.Hq // cfg.Hkv
    rec = []
    for kvh in range(cfg.Hkv):
        for j in range(8):
            qh = kvh * G + int(rng.integers(G))
            t = int(rng.integers(steps))
            p = int(rng.integers(0, n - 2 * cfg.block))
            qt = q[0, qh, t]
            k[0, kvh, p] = 4.0 * qt / np.linalg.norm(qt)
            v[0, kvh, p] = 0.0
            v[0, kvh, p, j] = 1.0
            rec.append((kvh, qh, n + t, p))
    q, k, v = (round_to(x, cfg.dtype) for x in (q, k, v))
    return {"cfg": cfg, "n_cache": n, "steps": steps, "q": q, "k": k, "v": v,
            "needles": np.array(rec, dtype=np.int64)}
