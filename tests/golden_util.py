"""Helpers shared by the CPU and GPU parity tests: golden fixture loading and the selection
comparison with its float32 tie certificate."""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"
U32 = 2.0 ** -24  # float32 unit roundoff


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# ssa_swap.ssa_masked fixtures: name -> (seed, (b, h, n, d), block, top_c, local)
MASKED_CASES = {
    "swap_masked_b16": (5, (2, 3, 300, 64), 16, 3, 1),
    "swap_masked_b64": (6, (1, 2, 200, 64), 64, 1, 0),
}


def masked_inputs(seed, b, h, n, d):
    """q, k, v and the upstream gradient g (b, h, n, d) float32 of an ssa_masked fixture."""
    rng = np.random.default_rng(seed)
    q, k, v, g = (rng.standard_normal((b, h, n, d)).astype(np.float32) for _ in range(4))
    return q, k, v, g


def row_sets(kv_num, kv_idx):
    kv_num = np.asarray(kv_num)
    kv_idx = np.asarray(kv_idx)
    flat_n = kv_num.reshape(-1)
    flat_i = kv_idx.reshape(-1, kv_idx.shape[-1])
    return [frozenset(int(c) for c in flat_i[r, :flat_n[r]]) for r in range(flat_n.size)]


def compare_selections(got_num, got_idx, ref_num, ref_idx, r64=None, mag=None, d=64,
                       mult=2.0):
    """Compares two compact selections row by row.

    Returns (n_rows, n_equal, n_certified, bad): rows whose sets differ are `certified` when
    every swapped pair (x taken only by ref, y taken only by got) has exact scores within the
    float32 evaluation noise of the reference: |r64[y] - r64[x]| <= mult * (d + 8) * u * mag, with
    mag the row's magnitude sum |q||mu| + c2 q^2 |var| (a worst-case bound on a length-d float32
    dot product). `bad` lists (row, ref-only, got-only) of uncertified differences.
    """
    gs = row_sets(got_num, got_idx)
    rs = row_sets(ref_num, ref_idx)
    assert len(gs) == len(rs), (len(gs), len(rs))
    nbk = None if r64 is None else r64.shape[-1]
    r64f = None if r64 is None else r64.reshape(-1, nbk)
    magf = None if mag is None else mag.reshape(-1, nbk)
    n_eq = n_cert = 0
    bad = []
    tol_rel = mult * (d + 8) * U32
    for row, (g, r) in enumerate(zip(gs, rs)):
        if g == r:
            n_eq += 1
            continue
        ref_only, got_only = sorted(r - g), sorted(g - r)
        ok = r64f is not None and len(ref_only) == len(got_only) and len(ref_only) > 0
        if ok:
            for x in ref_only:
                for y in got_only:
                    tol = tol_rel * max(magf[row, x], magf[row, y])
                    if abs(r64f[row, y] - r64f[row, x]) > tol:
                        ok = False
        if ok:
            n_cert += 1
        else:
            bad.append((row, ref_only, got_only))
    return len(gs), n_eq, n_cert, bad
