#!/usr/bin/env python3
"""Benchmark of the routed block-sparse attention hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--variant segmented|literal]

Headline workload ("C3"): one causal routed-prefill attention layer
at the Qwen2.5-0.5B attention shape -- 14 query / 2 key heads, d = 64, n = 131072, bf16,
block 128, top_c 64 + 2-block local window, beta 2. A step is the whole hot path over the
resident inputs: query-block means + key-block mean/variance -> cumulant router -> V transpose
-> block-sparse flash attention. value = n * K / (time of K steps) tokens/s.

Also reported on the same line: per-kernel times (HIP events on the stream the kernels run on),
the roofline of the dominant kernel (selected-block FLOPs = 4*b^2*d*sum(kv_num) per launch
against the 2.5 PFLOP/s bf16 dense MFMA peak; HBM traffic from the committed rocprofv3 PMC
summary when present), the dense causal baseline (torch SDPA) and this kernel at full budget,
the routed decode step at a 1M-token cache ("C4", ms/step), and the CPU baseline: the
reference's path restated in torch float32 (oracle/cpu_path.py) on this host's cores -- the C3
router in full, attention on a stated sample, C4 decode steps.

Only one GPU is used: --gpus N > 1 exits with a message.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "routed prefill tokens/s @128K (Qwen-0.5B shape); decode ms/step @1M ctx"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
PEAK_FP64_TFLOPS = 78.6


def router_fields(Hq, Hkv, nb, d, ms):
    """Budget-mode router work at Hq/Hkv heads over nb blocks: the reference einsum's FLOPs
    (2 * 2d per routable pair, row i against blocks c < i) and the bf16 MFMA FLOPs the score kernel
    issues: per key head, the Hq/Hkv heads' rows in 64-row tiles against the 64-candidate tiles
    below the tile's last row, three products per pair and head dim."""
    G = Hq // Hkv
    flops = 2.0 * (2 * d) * Hq * nb * (nb - 1) / 2
    R = G * nb
    tiles = 0
    for r0 in range(0, R, 64):
        r_last = min(r0 + 63, R - 1)
        imax = nb - 1 if r0 // nb != r_last // nb else r_last % nb
        tiles += -(-imax // 64)
    mfma = 3.0 * 2.0 * (2 * d) * 64 * 64 * tiles * Hkv
    s = ms / 1e3
    return {"ms": ms, "flops": flops, "mfma_flops": mfma, "tflops": flops / s / 1e12,
            "mfma_tflops": mfma / s / 1e12,
            # the reference einsum's FLOPs over the route time (the fraction of the bf16 peak the
            # router's algorithmic work reaches), and the issued bf16-split MFMA work's fraction
            "frac_bf16_peak_algorithmic": flops / s / 1e12 / PEAK_BF16_TFLOPS,
            "frac_bf16_mfma_peak": mfma / s / 1e12 / PEAK_BF16_TFLOPS,
            "method": "bf16-split MFMA scores, certified; band ranked by exact fp64 scores"}
IVF_NPROBE = 4          # build_ivf's default (ssa/ivf_kernel.py:63)
# the timed attention calls walk each workgroup's key blocks from a clock-derived position
# (sparse_attention(rotate=True): workgroups resident together share the key blocks they read
# in L2); outputs differ from the default list-order walk by fp32 rounding only
ROTATE = True
TRAFFIC_FILE = ROOT / "profiles" / "sparse_attn_c3_traffic.txt"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _event_ms(torch, fn, reps, warm=2):
    """Mean HIP-event time of fn() over reps calls on the current stream (after warm calls)."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


# paper/figures/ccc_kernel.json rows (RTX 4080): append / route / attention ms, certified rate
CCC_REFERENCE = {
    262144: {"append_ms": 2.717, "route_ms": 4.805, "attention_ms": 1.15, "cert_rate": 1.0},
    1048576: {"append_ms": 192.061, "route_ms": 60.818, "attention_ms": 5.128,
              "cert_rate": 0.968},
    4194304: {"append_ms": 132.086, "route_ms": 144.412, "attention_ms": 20.35,
              "cert_rate": 0.856},
    12582912: {"append_ms": 393.929, "route_ms": 519.643, "attention_ms": 66.802,
               "cert_rate": 0.737}}


def ccc_decompose(torch, dev, n, g, chunk_blocks=1024):
    """The reference's selector-share decomposition (ssa/cascade_router.py:459-503,
    decompose_ccc): clustered single-head keys and queries as its _gen (:459-473), one streaming
    pass of append (summaries, outliers, index upkeep) and route (search, certificate,
    escalation) per chunk of 1024 blocks, each timed between device synchronisations as the
    reference times them, then the block-sparse attention over the assembled lists."""
    from ssa_amd import cascade_router as CR, ssa_kernel as K
    d, blk = 64, 128
    nb4 = n // 32
    nc = max(8, int(nb4 ** 0.5))
    ctr = torch.randn(nc, d, generator=g, device=dev)
    a = torch.randint(0, nc, (nb4,), generator=g, device=dev)
    k = (ctr[a].repeat_interleave(32, 0) + 0.1 * torch.randn(n, d, generator=g, device=dev)).half()
    nbq = n // blk
    qc = ctr[torch.randint(0, nc, (nbq,), generator=g, device=dev)]
    q = (qc.repeat_interleave(blk, 0) + 0.2 * torch.randn(n, d, generator=g, device=dev)).half()
    v = torch.randn(n, d, generator=g, device=dev, dtype=torch.float16)
    del ctr, a, qc
    cc = CR.CausalCascade(d, block=blk, n_hint=n, chunk_blocks=chunk_blocks)
    W = min(cc.top_c + cc.local + 1 + cc.outlier_cap, nbq)
    kv_num = torch.empty(1, 1, nbq, dtype=torch.int32, device=dev)
    kv_idx = torch.zeros(1, 1, nbq, W, dtype=torch.int32, device=dev)
    cb = chunk_blocks * blk
    app = rte = 0.0
    certs, rounds, rebuilds = [], [], 0
    torch.cuda.synchronize()
    for t in range(0, n, cb):
        e = min(n, t + cb)
        before = cc.committed_at_rebuild
        t0 = time.perf_counter()
        cc.append(k[t:e])
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        kn, ki, cert, st = cc.route(q[t:e], t, certify=True)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        app += t1 - t0
        rte += t2 - t1
        rebuilds += cc.committed_at_rebuild != before and t > 0
        kv_num[0, 0, t // blk:e // blk] = kn
        kv_idx[0, 0, t // blk:e // blk, :ki.shape[1]] = ki
        certs.append(cert.float().mean().item())
        rounds.append(st["rounds"].float().mean().item())
    q4, k4, v4 = (x.view(1, 1, n, d) for x in (q, k, v))
    att = _event_ms(torch, lambda: K.sparse_attention(q4, k4, v4, kv_num, kv_idx, blk), 3, warm=1)
    sel = (app + rte) * 1000.0
    res = {"append_ms": app * 1000.0, "route_ms": rte * 1000.0, "attention_ms": att,
           "selector_share": sel / (sel + att), "rebuilds": rebuilds,
           "cert_rate": sum(certs) / len(certs), "mean_rounds": sum(rounds) / len(rounds),
           "sum_kv_num": int(kv_num.sum())}
    del q, k, v, q4, k4, v4, cc, kv_num, kv_idx
    torch.cuda.empty_cache()
    return res


def published_bench(torch, dev):
    """The shapes of the reference's own published measurements, run here with seeded N(0,1)
    inputs on the device. The reference's figures were taken on an RTX 4080 with FlexAttention /
    faiss-gpu: the ratios compare whole systems on different hardware, not kernels.
      flat-router SSA forward (ssa_flex: block_route + attention), B=1, H=8, d=64, fp16, block
        128, top_c 8, local 1, against dense SDPA causal: paper/figures/kernel_speed_measured.json
        :32-43 (13.25 / 203.9 ms at 131,072; 36.4 / 807 ms at 262,144);
      IVF-routed forward (ssa_flex_ivf), H=1, fp16, block 128, top_c 8:
        paper/figures/ivf_kernel_e2e.json:51-67,119-135 (16.1 ms at 1M, 139.5 ms at 12,582,912);
      routed decode step over a 1,048,576-token cache, H=1, fp16, block 128, top_c 8, local 1,
        mean of 128 steps: paper/figures/ivf_decode.json:17-31 (0.60 ms; dense 0.52 ms);
      treecode router (ssa/treecode_bench.py: build_tree over fp16 keys, H=8, d=64, block 128, F 8,
        then the Q-tiled descend_beam of nb random query rows per head, W 16, top_c 8):
        paper/figures/treecode_router_measured.json:18-33 (build 23.8 / descend 63.3 ms at
        1,048,576; 56.6 / 115.4 ms at 2,097,152);
      certified causal cascade (ccc_decompose below), H=1, d=64, clustered keys, certify,
        chunk_blocks 1024: paper/figures/ccc_kernel.json rows (append / route / attention)."""
    from ssa_amd import ivf_decode as D, ivf_kernel as IV, ssa_kernel as K, treecode as TC
    sdpa = torch.nn.functional.scaled_dot_product_attention
    g = torch.Generator(device=dev).manual_seed(11)

    def qkv(h, n):
        return [torch.randn(1, h, n, 64, device=dev, dtype=torch.float16, generator=g)
                for _ in range(3)]

    out = {"note": "reference_*: RTX 4080 figures (BASELINE.md section 1)"}
    for n, ref_ms, ref_dense in ((131072, 13.25, 203.9), (262144, 36.4, 807.0)):
        q, k, v = qkv(8, n)
        ms = _event_ms(torch, lambda: K.ssa_flex(q, k, v, 128, 8, 1), 5)
        dms = _event_ms(torch, lambda: sdpa(q, k, v, is_causal=True), 3, warm=1)
        out[f"flat_forward_h8_n{n}"] = {
            "ms": ms, "dense_sdpa_ms": dms, "speedup_vs_dense": dms / ms,
            "reference_ms": ref_ms, "reference_dense_ms": ref_dense,
            "reference_speedup_vs_dense": ref_dense / ref_ms}
        del q, k, v
    for n, ref_ms in ((1 << 20, 16.1), (12582912, 139.5)):
        q, k, v = qkv(1, n)
        ms = _event_ms(torch, lambda: IV.ssa_flex_ivf(q, k, v, 128, 8, 1), 3, warm=1)
        out[f"ivf_forward_h1_n{n}"] = {"ms": ms, "reference_ms": ref_ms}
        del q, k, v
    for n, ref_build, ref_desc in ((1 << 20, 23.832, 63.286), (1 << 21, 56.604, 115.384)):
        k = torch.randn(1, 8, n, 64, device=dev, dtype=torch.float16, generator=g)
        nb = n // 128
        qb = torch.randn(8, nb, 64, device=dev, generator=g)
        bms = _event_ms(torch, lambda: TC.build_tree(k, 128, 8), 3, warm=1)
        levels, F = TC.build_tree(k, 128, 8)
        dms_t = _event_ms(torch, lambda: TC.tree_router(levels, F, qb, 16, 8), 3, warm=1)
        out[f"treecode_h8_n{n}"] = {"build_ms": bms, "descend_ms": dms_t,
                                    "reference_build_ms": ref_build,
                                    "reference_descend_ms": ref_desc}
        del k, qb, levels
    ccc_decompose(torch, dev, 1 << 17, g)  # the cascade kernels' first launches, not reported
    for n, ref in CCC_REFERENCE.items():
        out[f"ccc_h1_n{n}"] = dict(ccc_decompose(torch, dev, n, g), reference=ref)
    n, steps = 1 << 20, 128
    q, k, v = qkv(1, n + steps)
    dec = D.RoutedDecoder(1, 1, 1, 64, n + steps, block=128, top_c=8, local=1,
                          dtype=torch.float16, device=dev)
    dec.prefill(k[:, :, :n], v[:, :, :n])
    o = torch.empty(1, 1, 64, device=dev, dtype=torch.float16)
    for t in range(8):
        dec.step(q[:, :, n + t], k[:, :, n + t], v[:, :, n + t], out=o)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(8, steps):
        dec.step(q[:, :, n + t], k[:, :, n + t], v[:, :, n + t], out=o)
    torch.cuda.synchronize()
    dms = (time.perf_counter() - t0) / (steps - 8) * 1000.0
    qd = q[:, :, n + steps - 1:n + steps]
    dense = _event_ms(torch, lambda: sdpa(qd, k[:, :, :n + steps], v[:, :, :n + steps]), 10)
    out["decode_h1_1m"] = {"ms_per_step": dms, "dense_sdpa_ms": dense, "reference_ms": 0.60,
                           "reference_dense_ms": 0.52}
    del q, k, v, dec
    return out


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--variant", default="segmented", choices=["segmented", "literal"])
    ap.add_argument("--prewarm-s", type=float, default=0.5,
                    help="seconds of untimed C3 steps before the warmup steps (clock ramp-up)")
    ap.add_argument("--decode-steps", type=int, default=128)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense baselines")
    ap.add_argument("--no-decode", action="store_true", help="skip the C4 decode step")
    ap.add_argument("--no-c5", action="store_true", help="skip the C5 12M-token prefill")
    ap.add_argument("--no-swap", action="store_true",
                    help="skip the trainable swap (ssa_masked forward + backward)")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the whole-model prefill timing (Qwen2.5-0.5B architecture)")
    ap.add_argument("--no-published", action="store_true",
                    help="skip the reference's own published shapes (RTX 4080 numbers)")
    ap.add_argument("--swap-only", action="store_true",
                    help="run only the swap arm and print its JSON (for profiling)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (PMC byte-count calibration)")
    return ap.parse_args()


class Timer:
    """HIP-event timer on the current stream (where every ssa_amd kernel is launched)."""

    def __init__(self, torch):
        self.torch = torch
        self.acc = {}

    def run(self, name, fn, *a, **kw):
        t = self.torch
        s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        s.record()
        r = fn(*a, **kw)
        e.record()
        self.acc.setdefault(name, []).append((s, e))
        return r

    def mean_ms(self, name):
        ev = self.acc[name]
        return sum(s.elapsed_time(e) for s, e in ev) / len(ev)

    def reset(self):
        self.acc = {}


def read_traffic():
    """(HBM bytes per launch, L2 hit rate) of the attention kernel from the committed rocprofv3
    counter summary, or (None, None)."""
    if not TRAFFIC_FILE.exists():
        return None, None
    kv = {}
    for line in TRAFFIC_FILE.read_text().splitlines():
        if ":" in line and not line.lstrip().startswith("#"):
            key, val = line.split(":", 1)
            kv[key.strip()] = val.strip()
    try:
        traffic = float(kv["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        traffic = None
    try:
        hit, miss = float(kv["tcc_hit_per_launch"]), float(kv["tcc_miss_per_launch"])
        l2 = hit / (hit + miss)
    except (KeyError, ValueError, ZeroDivisionError):
        l2 = None
    return traffic, l2


def device_info(torch, dev):
    """The box's own figures: CU count and clock (rocminfo) -> derived bf16 MFMA peak, and the
    achievable HBM rates of a plain 2 GiB device copy and of a plain 2 GiB fill (write only)."""
    props = torch.cuda.get_device_properties(dev)
    info = {"name": props.name, "arch": getattr(props, "gcnArchName", ""),
            "cus": props.multi_processor_count}
    try:
        import re
        import subprocess
        txt = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=60).stdout
        clocks = [int(m.group(1)) for agent in re.split(r"\n\*+\s*\nAgent \d+", txt)
                  if re.search(r"Device Type:\s+GPU", agent)
                  for m in [re.search(r"Max Clock Freq\. \(MHz\):\s+(\d+)", agent)] if m]
        gpu_clk = max(clocks) if clocks else None
    except (OSError, subprocess.SubprocessError):
        gpu_clk = None
    if gpu_clk:
        info["max_sclk_mhz"] = gpu_clk
        # gfx950: 4 SIMDs x 1024 bf16 FLOP per clock per SIMD (dense MFMA)
        info["bf16_mfma_peak_derived_tflops"] = props.multi_processor_count * 4096 * gpu_clk / 1e6
    src = torch.empty(1 << 31, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    gbs = 2 * src.numel() * 5 / (time.perf_counter() - t0) / 1e9
    info["hbm_copy_gbs"] = gbs
    info["hbm_copy_frac_of_8tbs"] = gbs / PEAK_HBM_GBS
    # write-only rate (a plain fill of the same 2 GiB): what a kernel that mostly stores can reach
    for _ in range(2):
        dst.fill_(1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        dst.fill_(1)
    torch.cuda.synchronize()
    info["hbm_fill_gbs"] = src.numel() * 5 / (time.perf_counter() - t0) / 1e9
    del src, dst
    # the MFMA rate a plain library GEMM sustains on this box (hipBLASLt through torch.matmul,
    # bf16 8192^3): the practical ceiling the attention kernels' roofline fraction compares with
    a = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
    b = torch.randn(8192, 8192, device=dev, dtype=torch.bfloat16)
    c = torch.empty(8192, 8192, device=dev, dtype=torch.bfloat16)
    for _ in range(3):
        torch.matmul(a, b, out=c)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        torch.matmul(a, b, out=c)
    e1.record()
    torch.cuda.synchronize()
    tf = 2.0 * 8192 ** 3 * 10 / (e0.elapsed_time(e1) * 1e-3) / 1e12
    info["gemm_bf16_8192_tflops"] = tf
    info["gemm_bf16_frac_of_peak"] = tf / PEAK_BF16_TFLOPS
    del a, b, c
    return info


def cpu_threads(torch):
    """Host threads for the CPU baseline: the cores this process may use (OMP_NUM_THREADS caps
    it where set, as on the GPU boxes)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    torch.set_num_threads(n)
    return torch.get_num_threads()


def _runs(fn, runs):
    """Wall-clock seconds of `runs` calls of fn."""
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return ts


def _med_iqr(ts):
    """{median_s, iqr_s, runs} of a list of run times."""
    import numpy as np
    q1, med, q3 = np.percentile(np.asarray(ts, dtype=np.float64), [25, 50, 75])
    return {"median_s": float(med), "iqr_s": float(q3 - q1), "runs": len(ts)}


def _cpu_prefill_full(C, torch, p, runs):
    """Router + block-sparse softmax of every (head, query block) pair of a config, on the host.
    Returns (run times, kv_num)."""
    cfg = p["cfg"]
    dt = torch.float32 if cfg.dtype == torch.float32 else torch.bfloat16
    q, k, v = (torch.from_numpy(p[x]).to(dt) for x in ("q", "k", "v"))
    pairs = [(h, i) for h in range(cfg.Hq) for i in range(cfg.nb)]
    res = {}

    def once():
        kv_num, kv_idx, _ = C.route_budget(q, k, cfg.block, top_c=cfg.top_c, local=cfg.local,
                                           beta=cfg.beta)
        C.attend_blocks(q, k, v, kv_num, kv_idx, cfg.block, pairs)
        res["kv_num"] = kv_num
    return _runs(once, runs), res["kv_num"]


def cpu_baseline(p, dec, c5=None):
    """The reference's path restated in torch float32 on this host's cores (oracle/cpu_path.py;
    ssa/ssa_kernel.py:61-119 and the FlexAttention softmax, ssa/ivf_decode.py:49-62 with the
    router of ssa/gemma_ssa.py:99-131), each part as the median and inter-quartile range of
    repeated runs:
      c1, c2  router + attention in full (5 and 3 runs);
      c3      the router in full and attention over a stratified sample of (query head, query
              block) pairs (every query block once, heads in turn), extrapolated by sum(kv_num)
              (3 runs each) -- the headline `value`;
      c4      decode steps over the full 1,048,576-token cache (3 runs of 8 steps);
      c5      (from the C5 arm) the router over a prefix of the query blocks, extrapolated by the
              square of the block count (its score matrix and top-k grow with nb^2), and
              attention over 32 evenly spaced query blocks, extrapolated by sum(kv_num)."""
    import torch

    from oracle import cpu_path as C
    from ssa_amd import workloads as WL
    threads = cpu_threads(torch)
    cfg = p["cfg"]
    q, k, v = (torch.from_numpy(p[x]).to(torch.bfloat16) for x in ("q", "k", "v"))
    res = {}

    def route():
        res["r"] = C.route_budget(q, k, cfg.block, top_c=cfg.top_c, local=cfg.local, beta=cfg.beta)
    t_route = _runs(route, 3)
    kv_num, kv_idx, _ = res["r"]
    nb = cfg.nb
    pairs = [(i % cfg.Hq, i) for i in range(nb)]  # every query block once, heads in turn
    sample_kv = sum(int(kv_num[0, h, i]) for h, i in pairs)
    total_kv = int(kv_num.sum())
    t_sample = _runs(lambda: C.attend_blocks(q, k, v, kv_num, kv_idx, cfg.block, pairs), 3)
    route_s, sample_s = _med_iqr(t_route), _med_iqr(t_sample)
    t_attn = sample_s["median_s"] * total_kv / sample_kv
    t_total = route_s["median_s"] + t_attn
    out = {
        "value": cfg.n / t_total, "unit": "tokens/s", "cores": threads, "kind": "port",
        "sample": (f"C3: torch fp32 host restatement (oracle/cpu_path.py): router over all "
                   f"{cfg.Hq * nb} rows + softmax on {len(pairs)} (head, q-block) pairs "
                   f"({100.0 * sample_kv / total_kv:.2f} % of tiles), scaled by sum(kv_num); "
                   f"medians of 3 runs"),
        "c3": {"router": route_s, "attention_sample": sample_s,
               "attention_s_extrapolated": t_attn, "sample_fraction": sample_kv / total_kv,
               "tokens_per_s": cfg.n / t_total},
    }
    del q, k, v, res
    for name, runs in (("C1", 5), ("C2", 3)):
        pc = WL.make(name)
        ts, _ = _cpu_prefill_full(C, torch, pc, runs)
        st = _med_iqr(ts)
        out[name.lower()] = dict(st, workload=f"{name} router + attention in full",
                                 tokens_per_s=pc["cfg"].n / st["median_s"])
        del pc
    if dec is not None:
        c4 = dec["cfg"]
        n0 = dec["n_cache"]
        kc = torch.from_numpy(dec["k"][0]).to(torch.bfloat16)
        vc = torch.from_numpy(dec["v"][0]).to(torch.bfloat16)
        qd = torch.from_numpy(dec["q"][0]).to(torch.bfloat16)  # (Hq, steps, d)
        ncomp = (n0 + 8) // c4.block
        kb = kc[:, :ncomp * c4.block].float().reshape(c4.Hkv, ncomp, c4.block, c4.d)
        mu, var = kb.mean(2), kb.var(2, unbiased=False)  # resident summaries (not timed)
        del kb

        def steps8():
            for t in range(8):
                C.decode_step(qd[:, t], kc, vc, mu, var, n0 + t, c4.block, c4.top_c, c4.local,
                              c4.beta)
        st = _med_iqr([x / 8 for x in _runs(steps8, 3)])
        out["c4"] = {"ms_per_step": st["median_s"] * 1e3, "iqr_ms": st["iqr_s"] * 1e3,
                     "runs": st["runs"],
                     "workload": f"{c4.Hq} heads, {n0}-token cache, 3 runs of 8 steps"}
    if c5 is not None:
        out["c5"] = c5
    return out


def cpu_baseline_c5(torch, c5, q5, k5, v5, kn5, ki5, prefix_blocks=4096, sample_blocks=32):
    """C5 on the host (see cpu_baseline): router over the first `prefix_blocks` query blocks
    (their causal past is inside the prefix) and attention over `sample_blocks` evenly spaced
    query blocks with the device router's lists, each extrapolated and labelled so."""
    import numpy as np

    from oracle import cpu_path as C
    cpu_threads(torch)
    nb = c5.n // c5.block
    npre = prefix_blocks * c5.block
    qp = q5[:, :, :npre].cpu()
    kp = k5[:, :, :npre].cpu()
    t_route = _med_iqr(_runs(lambda: C.route_budget(qp, kp, c5.block, top_c=c5.top_c,
                                                    local=c5.local, beta=c5.beta), 3))
    del qp, kp
    qh, kh, vh = q5.cpu(), k5.cpu(), v5.cpu()
    num, idx = kn5.cpu(), ki5.cpu()
    rows = np.linspace(0, nb - 1, sample_blocks).astype(np.int64).tolist()
    pairs = [(0, i) for i in rows]
    sample_kv = sum(int(num[0, 0, i]) for i in rows)
    total_kv = int(num.sum())
    t_attn = _med_iqr(_runs(lambda: C.attend_blocks(qh, kh, vh, num, idx, c5.block, pairs), 3))
    del qh, kh, vh
    route_x = t_route["median_s"] * (nb / prefix_blocks) ** 2
    attn_x = t_attn["median_s"] * total_kv / sample_kv
    return {"router_prefix": t_route, "router_s_extrapolated": route_x,
            "attention_sample": t_attn, "attention_s_extrapolated": attn_x,
            "tokens_per_s": c5.n / (route_x + attn_x),
            "sample": (f"router over the first {prefix_blocks} of {nb} query blocks, scaled by "
                       f"({nb}/{prefix_blocks})^2; attention over {sample_blocks} evenly spaced "
                       f"query blocks ({100.0 * sample_kv / total_kv:.3f} % of tiles), scaled by "
                       f"sum(kv_num); medians of 3 runs")}


def swap_bench(torch, dev):
    """ssa_swap.ssa_masked training step at the reference's swap configuration (GPT-2 attention:
    batch 4, 12 heads, context 1024, d 64, fp32; block 64, top_c 4, local 2): router, forward and
    backward on HIP events, against torch SDPA dense causal forward + backward; also in bf16."""
    from ssa_amd import ssa_swap as S
    out = {"workload": "ssa_masked training step: B=4, H=12, n=1024, d=64 (GPT-2 attention), "
                       "block 64, top_c 4, local 2; q/k/v ~ N(0,1)"}
    for dt, tag in ((torch.float32, "fp32"), (torch.bfloat16, "bf16")):
        g = torch.Generator(device=dev).manual_seed(0)
        q, k, v, go = (torch.randn(4, 12, 1024, 64, device=dev, dtype=dt, generator=g)
                       for _ in range(4))
        for t in (q, k, v):
            t.requires_grad_(True)
        tm = Timer(torch)
        for rep in range(8):
            tmr = tm if rep >= 3 else Timer(torch)
            kv_num, kv_idx = tmr.run("route", S.route_masked, q.detach(), k.detach(), 64, 4, 2)
            o = tmr.run("fwd", S._MaskedAttention.apply, q, k, v, kv_num, kv_idx, 64, 0.125)
            tmr.run("bwd", o.backward, go)
            q.grad = k.grad = v.grad = None
            d_o = tmr.run("sdpa_fwd", torch.nn.functional.scaled_dot_product_attention, q, k, v,
                          is_causal=True)
            tmr.run("sdpa_bwd", d_o.backward, go)
            q.grad = k.grad = v.grad = None
        torch.cuda.synchronize()
        ms = {x: tm.mean_ms(x) for x in ("route", "fwd", "bwd", "sdpa_fwd", "sdpa_bwd")}
        total = ms["route"] + ms["fwd"] + ms["bwd"]
        dense = ms["sdpa_fwd"] + ms["sdpa_bwd"]
        out[tag] = {**{f"{x}_ms": y for x, y in ms.items()}, "step_ms": total,
                    "sdpa_step_ms": dense, "speedup_vs_sdpa": dense / total,
                    "mean_blocks_per_row": float(kv_num.float().mean().item())}
        del q, k, v, go, o, d_o
    return out


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "bench.py runs on exactly one GPU: this build has no "
                          "multi-GPU path (one MI355X box has one GPU); run with --gpus 1"}))
        sys.exit(2)

    import numpy as np
    import torch

    from ssa_amd import _lib
    from ssa_amd import ivf_decode as D
    from ssa_amd import ivf_kernel as IV
    from ssa_amd import ssa_kernel as K
    from ssa_amd import workloads as WL

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.swap_only:
        print(json.dumps({"swap": swap_bench(torch, dev)}), flush=True)
        return
    log("bench: generating C3 inputs")
    p = WL.make("C3", args.variant)
    cfg = p["cfg"]
    q, k, v = (WL.to_device(p[x], cfg.dtype, dev) for x in ("q", "k", "v"))
    n, blk = cfg.n, cfg.block
    tm = Timer(torch)

    # the attention call's workspace, reused step after step: prepare_attention writes V^T, the
    # fp16 key copy and the per-tile key-norm maxima into it in one pass over K and V
    ws_attn = torch.empty(int(_lib.query("ssa_sparse_attn_workspace_size", _lib.dtype_code(v.dtype),
                                         1, cfg.Hkv, n, cfg.d, blk)), device=dev, dtype=torch.uint8)

    def step(timer):
        qbar = timer.run("qmean", K.block_summary, q, blk, "qmean")
        mu, var, _ = timer.run("kstats", K.block_summary, k, blk, "pop")
        kv_num, kv_idx = timer.run("route", K.route, qbar, mu, var, None, "budget", cfg.top_c,
                                   0.0, cfg.local, 0.5 * cfg.beta)
        prep = timer.run("prepare_kv", K.prepare_attention, k, v, blk, ws_attn)
        out = timer.run("attention", K.sparse_attention, q, k, v, kv_num, kv_idx, blk,
                        prepared=prep, rotate=ROTATE)
        return out, kv_num

    # The GPU raises its clocks over the first ~40 ms of sustained load (the attention launches
    # of a fresh process run 5.2 -> 3.8 ms over their first ~8 calls), so the device is brought
    # to its steady state with untimed steps for --prewarm-s seconds before the W warmup steps;
    # the K timed steps are unchanged.
    log(f"bench: prewarm {args.prewarm_s} s, warmup {args.warmup}")
    pw = Timer(torch)
    t_pw = time.perf_counter()
    while time.perf_counter() - t_pw < args.prewarm_s:
        step(pw)
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        out, kv_num = step(tm)
    torch.cuda.synchronize()
    tm.reset()
    log(f"bench: timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out, kv_num = step(tm)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall / args.steps * 1000.0
    parts = {nm: tm.mean_ms(nm) for nm in ("qmean", "kstats", "route", "prepare_kv", "attention")}
    sum_kv = int(kv_num.sum().item())
    flops = 4.0 * blk * blk * cfg.d * sum_kv
    t_attn = parts["attention"] / 1e3
    achieved = flops / t_attn / 1e12
    traffic, l2_hit = read_traffic()
    diag = cfg.Hq * cfg.nb
    flops_causal = 4.0 * cfg.d * (blk * blk * (sum_kv - diag) + diag * blk * (blk + 1) / 2)
    summary_bytes = (cfg.Hkv + cfg.Hq) * n * cfg.d * 2 + (2 * cfg.Hkv + cfg.Hq) * cfg.nb * cfg.d * 4
    log(f"bench: {ms_step:.3f} ms/step; parts {parts}; sum kv_num {sum_kv}")
    # the same attention call with every workgroup on the exact path (fp32-scaled scores, running
    # max): what rows beyond the bounded path's +-32 log2-unit admission bound run at
    te = Timer(torch)
    qbar = K.block_summary(q, blk, "qmean")
    mu, var, _ = K.block_summary(k, blk, "pop")
    enum_, eidx = K.route(qbar, mu, var, None, "budget", cfg.top_c, 0.0, cfg.local, 0.5 * cfg.beta)
    for i in range(12):
        prep = K.prepare_attention(k, v, blk, ws_attn)
        te.run("exact" if i >= 2 else "warm", K.sparse_attention, q, k, v, enum_, eidx, blk,
               prepared=prep, exact=True)
    torch.cuda.synchronize()
    exact_ms = te.mean_ms("exact")
    del qbar, mu, var, enum_, eidx

    result = {
        "metric": METRIC, "value": n / (ms_step / 1e3), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "prewarm_s": args.prewarm_s,
        "ms_per_step": ms_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": f"synthetic: seeded NumPy PCG64 (seed {cfg.seed}), keys from a 256-component "
                f"Gaussian mixture ({args.variant}), Q/V ~ N(0,1), resident in HBM",
        "config": {"workload": "C3: one causal routed-prefill attention layer, Qwen2.5-0.5B "
                               "attention shape (14q/2kv heads, d=64), n=131072, block 128, "
                               "top_c 64 + local 2, beta 2, summaries+router+attention per step",
                   "n": n, "Hq": cfg.Hq, "Hkv": cfg.Hkv, "d": cfg.d, "block": blk,
                   "top_c": cfg.top_c, "local": cfg.local, "beta": cfg.beta,
                   "variant": args.variant},
        "roofline": {"bound": "mfma", "kernel": "sparse_attn_dma_kernel",
                     "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_BF16_TFLOPS, "traffic": traffic,
                     # the same time with the masked upper halves of the diagonal tiles not
                     # counted (the causal-exact FLOPs)
                     "frac_causal_exact": flops_causal / t_attn / 1e12 / PEAK_BF16_TFLOPS,
                     "attention_walk": "clock-rotated" if ROTATE else "list order",
                     "traffic_source": f"committed profile {TRAFFIC_FILE.name}",
                     "flops_per_launch": flops, "flops_causal_exact": flops_causal,
                     "sum_kv_num": sum_kv, "l2_hit_rate": l2_hit,
                     "gathered_kv_bytes": sum_kv * 2 * blk * cfg.d * 2},
        "breakdown_ms": parts,
        "exact_path": {"attention_ms": exact_ms, "tflops": flops / (exact_ms / 1e3) / 1e12,
                       "frac": flops / (exact_ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS,
                       "note": "sparse_attention(exact=True): every workgroup on the exact path"},
        "summaries_gbs": summary_bytes / ((parts["qmean"] + parts["kstats"]) / 1e3) / 1e9,
        "summaries": {"bytes": summary_bytes, "ms": parts["qmean"] + parts["kstats"],
                      "hbm_frac": summary_bytes / ((parts["qmean"] + parts["kstats"]) / 1e3)
                      / 1e9 / PEAK_HBM_GBS},
        # the router scores on bf16 MFMA (each fp32 product as three bf16 products of a hi/lo
        # split) and certifies its selection, ranking the error band exactly; "flops" counts the
        # reference's einsum (2 * 2d per routable pair), "mfma_flops" what the score kernel
        # issues (its 64 x 64 tiles, three products each); ms is the whole route (score + select)
        "router": router_fields(cfg.Hq, cfg.Hkv, cfg.nb, cfg.d, parts["route"]),
    }
    result["device"] = device_info(torch, dev)

    # the IVF router (f4) at the headline shape, after the timed steps: each key head's index
    # serves its 7 query heads; compared with the flat router's time above
    ti = Timer(torch)
    nb3 = cfg.n // blk
    qb3 = K.block_summary(q, blk, "qmean").view(cfg.Hq, nb3, cfg.d)
    mu3 = K.block_summary(k, blk, "pop")[0].view(cfg.Hkv, nb3, cfg.d)
    for rep in range(4):
        tmr = ti if rep else Timer(torch)
        idx3 = tmr.run("ivf_build", IV.build_ivf, mu3, None, IVF_NPROBE)
        tmr.run("ivf_route", IV.search, idx3, qb3, cfg.top_c, cfg.local, IVF_NPROBE,
                2 * cfg.top_c)
    torch.cuda.synchronize()
    result["c3_ivf"] = {
        "note": "approximate IVF router timing; selections differ from the exact router's",
        "router": f"IVF over each key head's {nb3} block means: nlist {idx3.nlist}, nprobe "
                  f"{IVF_NPROBE}, search_k {2 * cfg.top_c}, top_c {cfg.top_c} + local {cfg.local}",
        "build_ms": ti.mean_ms("ivf_build"), "route_ms": ti.mean_ms("ivf_route"),
        "flat_route_ms": parts["route"],
    }
    del idx3, qb3, mu3

    if not args.no_dense:
        log("bench: dense baselines")
        kr, vr = k.repeat_interleave(cfg.Hq // cfg.Hkv, dim=1), v.repeat_interleave(cfg.Hq // cfg.Hkv, dim=1)
        sd = Timer(torch)
        for i in range(4):
            sd.run("sdpa" if i else "warm", torch.nn.functional.scaled_dot_product_attention,
                   q, kr, vr, is_causal=True)
        qbar = K.block_summary(q, blk, "qmean")
        mu, var, _ = K.block_summary(k, blk, "pop")
        fnum, fidx = K.route(qbar, mu, var, None, "budget", None, 1.0, cfg.local, 0.5 * cfg.beta)
        for i in range(3):
            prep = K.prepare_attention(k, v, blk, ws_attn)
            sd.run("own_full" if i else "warm", K.sparse_attention, q, k, v, fnum, fidx, blk,
                   prepared=prep, rotate=ROTATE)
        torch.cuda.synchronize()
        dense_ms = sd.mean_ms("sdpa")
        own_full = sd.mean_ms("own_full")
        dense_flops = 4.0 * cfg.d * cfg.Hq * n * (n + 1) / 2
        result["dense"] = {
            "sdpa_causal_ms": dense_ms, "own_kernel_full_budget_ms": own_full,
            "speedup_vs_sdpa": dense_ms / ms_step, "attention_speedup_vs_sdpa": dense_ms / parts["attention"],
            # the same kernel at full budget (every causal block): the routed call's speedup over
            # dense attention by this build's own kernel, bounded by the FLOP ratio
            "attention_speedup_vs_own_full_budget": own_full / parts["attention"],
            "sdpa_tflops": dense_flops / (dense_ms / 1e3) / 1e12,
            "own_full_tflops": 4.0 * blk * blk * cfg.d * int(fnum.sum().item()) / (own_full / 1e3) / 1e12,
        }
        del kr, vr

    dec_host = None
    c5_cpu = None
    if not args.no_decode:
        log("bench: C4 decode")
        ds = WL.make_decode(steps=args.decode_steps + 8)
        c4 = ds["cfg"]
        ncache = ds["n_cache"]
        dec = D.RoutedDecoder(1, c4.Hq, c4.Hkv, c4.d, ncache + args.decode_steps + 8,
                              block=c4.block, top_c=c4.top_c, local=c4.local, beta=c4.beta,
                              dtype=c4.dtype, device=dev)
        kd, vd = WL.to_device(ds["k"], c4.dtype, dev), WL.to_device(ds["v"], c4.dtype, dev)
        qd = WL.to_device(ds["q"], c4.dtype, dev)
        qd = qd.permute(2, 0, 1, 3).contiguous()  # (steps, B, Hq, d): each step's q contiguous
        dec.prefill(kd[:, :, :ncache], vd[:, :, :ncache])
        out_d = torch.empty(1, c4.Hq, c4.d, device=dev, dtype=c4.dtype)
        for t in range(8):
            dec.step(qd[t], kd[:, :, ncache + t], vd[:, :, ncache + t], out=out_d)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in range(8, 8 + args.decode_steps):
            dec.step(qd[t], kd[:, :, ncache + t], vd[:, :, ncache + t], out=out_d)
        torch.cuda.synchronize()
        dms = (time.perf_counter() - t0) / args.decode_steps * 1000.0
        # the same steps captured in a HIP graph through the allocation-free entry point
        # (ssa_decode_step_static): 32 consecutive steps per graph (each with its position baked
        # in; a replay appends the same tokens again), replayed back to back
        decs = D.RoutedDecoder(1, c4.Hq, c4.Hkv, c4.d, ncache + args.decode_steps + 8,
                               block=c4.block, top_c=c4.top_c, local=c4.local, beta=c4.beta,
                               dtype=c4.dtype, device=dev, static_scratch=True)
        decs.prefill(kd[:, :, :ncache], vd[:, :, :ncache])
        for t in range(8):
            decs.step(qd[t], kd[:, :, ncache + t], vd[:, :, ncache + t], out=out_d)
        gs = torch.cuda.Stream()
        gs.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        ng = 32
        with torch.cuda.stream(gs):
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=gs):
                for t in range(8, 8 + ng):
                    decs.step(qd[t], kd[:, :, ncache + t], vd[:, :, ncache + t], out=out_d)
        torch.cuda.synchronize()
        for _ in range(2):
            graph.replay()
        torch.cuda.synchronize()
        reps = max(1, args.decode_steps // ng)
        t0 = time.perf_counter()
        for _ in range(reps):
            graph.replay()
        torch.cuda.synchronize()
        gms = (time.perf_counter() - t0) / (reps * ng) * 1000.0
        del graph, decs
        kvn = int(dec.kv_num.sum().item())
        nbk = dec.pos // c4.block
        dbytes = c4.Hkv * nbk * 2 * c4.d * 4 + kvn * c4.block * c4.d * 2 * 2
        # dense baseline (ssa/ivf_decode.py:65-74 at this shape): one SDPA call over the whole
        # cache prefix, the 7 query heads of a key head stacked as 7 query rows of it (no mask is
        # needed at decode, and K/V are read once, not repeated per query head)
        npre = dec.pos
        G4 = c4.Hq // c4.Hkv
        qd1 = qd[8].reshape(1, c4.Hkv, G4, c4.d)
        kpre, vpre = dec.kcache[:, :, :npre], dec.vcache[:, :, :npre]
        sdpa = torch.nn.functional.scaled_dot_product_attention
        for _ in range(3):
            sdpa(qd1, kpre, vpre)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(32):
            sdpa(qd1, kpre, vpre)
        torch.cuda.synchronize()
        dense_dms = (time.perf_counter() - t0) / 32 * 1000.0
        result["decode"] = {
            "workload": "C4: decode, bf16, 14q/2kv, d=64, 1M-token cache, block 128, top_c 64",
            "ms_per_step": dms, "steps": args.decode_steps,
            "graph_ms_per_step": gms,
            "graph": f"{ng} steps per HIP graph through ssa_decode_step_static, replayed {reps}x",
            "bytes_per_step": dbytes, "achieved_gbs": dbytes / (dms / 1e3) / 1e9,
            "hbm_frac": dbytes / (dms / 1e3) / 1e9 / PEAK_HBM_GBS,
            # torch SDPA has no split-KV decode path on ROCm: its grid is (query tiles x
            # heads), 2 workgroups here, so the HBM floor of a dense step is reported beside it
            "dense_sdpa_ms_per_step": dense_dms,
            "speedup_vs_dense_sdpa": dense_dms / dms,
            "dense_bytes_per_step": 2 * c4.Hkv * npre * c4.d * 2,
            "dense_hbm_floor_ms": 2 * c4.Hkv * npre * c4.d * 2 / (PEAK_HBM_GBS * 1e6),
            "speedup_vs_dense_hbm_floor": 2 * c4.Hkv * npre * c4.d * 2 / (PEAK_HBM_GBS * 1e6) / dms,
        }
        del kd, vd, qd, dec
        dec_host = ds

    if not args.no_swap:
        log("bench: attention swap (ssa_masked forward + backward)")
        result["swap"] = swap_bench(torch, dev)

    if not args.no_prefill:
        log("bench: whole-model prefill (Qwen2.5-0.5B architecture, random weights)")
        try:
            from ssa_amd import longctx_swap as L
            res = L.run([32768, 131072], [1.0, 0.25, 0.12, 0.06], log=log)
            res["workload"] = ("24-layer Qwen2.5-0.5B architecture, bf16, random weights, "
                               "YaRN x4; dense = SDPA, hip = install_ssa(impl='hip')")
            result["prefill"] = res
        except Exception as e:  # reported, never fatal to the headline line
            result["prefill"] = {"error": f"{type(e).__name__}: {e}"}
        torch.cuda.empty_cache()

    if not args.no_c5:
        log("bench: C5 12M-token prefill")
        del q, k, v
        torch.cuda.empty_cache()
        d5 = WL.make_c5_device(dev)
        c5 = d5["cfg"]
        q5, k5, v5 = d5["q"], d5["k"], d5["v"]
        nb5 = c5.n // c5.block
        ws5 = torch.empty(int(_lib.query("ssa_sparse_attn_workspace_size",
                                         _lib.dtype_code(v5.dtype), 1, 1, c5.n, c5.d, c5.block)),
                          device=dev, dtype=torch.uint8)
        t5 = Timer(torch)
        layer_ev = []
        for rep in range(4):
            tmr = t5 if rep else Timer(torch)
            # the flat-routed layer, also timed whole (first to last kernel) on its stream
            l0, l1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            l0.record()
            qb5 = tmr.run("summaries", K.block_summary, q5, c5.block, "qmean")
            mu5, var5, _ = tmr.run("summaries_k", K.block_summary, k5, c5.block, "pop")
            kn5, ki5 = tmr.run("route", K.route, qb5, mu5, var5, None, "budget", c5.top_c, 0.0,
                               c5.local, 0.5 * c5.beta)
            prep5 = tmr.run("prepare_kv", K.prepare_attention, k5, v5, c5.block, ws5)
            tmr.run("attention", K.sparse_attention, q5, k5, v5, kn5, ki5, c5.block,
                    prepared=prep5, rotate=ROTATE)
            vt5 = prep5.ws[:v5.numel() * 2].view(v5.dtype).view(1, 1, c5.d, nb5 * c5.block)
            l1.record()
            if rep:
                layer_ev.append((l0, l1))
            # the IVF router (sub-linear, approximate) on the same summaries, and the attention
            # over its lists
            idx5 = tmr.run("ivf_build", IV.build_ivf, mu5.view(1, nb5, c5.d), None, IVF_NPROBE)
            ivn, ivi = tmr.run("ivf_route", IV.search, idx5, qb5.view(1, nb5, c5.d), c5.top_c,
                               c5.local, IVF_NPROBE, 2 * c5.top_c)
            ivn4, ivi4 = ivn.view(1, 1, nb5), ivi.view(1, 1, nb5, -1)
            tmr.run("ivf_attention", K.sparse_attention, q5, k5, v5, ivn4, ivi4, c5.block, vt=vt5,
                    rotate=ROTATE)
        torch.cuda.synchronize()
        rows5 = np.linspace(c5.top_c, nb5 - 1, 256).astype(np.int64)
        kn_h, ki_h = kn5[0, 0].cpu().numpy(), ki5[0, 0].cpu().numpy()
        ivn_h, ivi_h = ivn[0].cpu().numpy(), ivi[0].cpu().numpy()
        jac5 = []
        for i in rows5:
            a = set(ki_h[i, :kn_h[i]].tolist())
            b = set(ivi_h[i, :ivn_h[i]].tolist())
            jac5.append(len(a & b) / max(1, len(a | b)))
        ivf_router = (t5.mean_ms("summaries") + t5.mean_ms("summaries_k") +
                      t5.mean_ms("ivf_build") + t5.mean_ms("ivf_route"))
        ivf_total = ivf_router + t5.mean_ms("prepare_kv") + t5.mean_ms("ivf_attention")
        router = t5.mean_ms("summaries") + t5.mean_ms("summaries_k") + t5.mean_ms("route")
        attn = t5.mean_ms("prepare_kv") + t5.mean_ms("attention")
        layer = sum(a.elapsed_time(b) for a, b in layer_ev) / len(layer_ev)
        kv5 = int(kn5.sum().item())
        result["c5"] = {
            "workload": "C5: 1 head, fp16, d=64, n=12,582,912, block 256, top_c 64 + local 1",
            "router_ms": router, "attention_ms": attn, "total_ms": layer,
            "tokens_per_s": c5.n / (layer / 1e3), "sum_of_parts_ms": router + attn,
            "note": "total_ms: the flat-routed layer on the GPU from its first to its last "
                    "kernel (HIP events); the parts are the kernels' own times",
            "summaries_ms": t5.mean_ms("summaries") + t5.mean_ms("summaries_k"),
            "route_ms": t5.mean_ms("route"), "attention_kernel_ms": t5.mean_ms("attention"),
            "router": router_fields(1, 1, nb5, c5.d, t5.mean_ms("route")),
            "attention_tflops": 4.0 * c5.block * c5.block * c5.d * kv5 / (t5.mean_ms("attention") / 1e3) / 1e12,
            "sum_kv_num": kv5,
            "ivf": {
                "note": "approximate IVF router timing, not a C5 result (Jaccard below)",
                "router": f"nlist {idx5.nlist}, nprobe {IVF_NPROBE}, search_k {2 * c5.top_c}",
                "build_ms": t5.mean_ms("ivf_build"), "route_ms": t5.mean_ms("ivf_route"),
                "router_ms": ivf_router, "attention_kernel_ms": t5.mean_ms("ivf_attention"),
                "total_ms": ivf_total, "tokens_per_s": c5.n / (ivf_total / 1e3),
                "router_speedup_vs_flat": router / ivf_router,
                "sum_kv_num": int(ivn.sum().item()),
                "jaccard_vs_flat_256_rows": float(np.mean(jac5)),
            },
        }
        if not args.no_cpu:
            log("bench: C5 CPU baseline (router prefix, attention sample)")
            c5_cpu = cpu_baseline_c5(torch, c5, q5, k5, v5, kn5, ki5)
        del q5, k5, v5, d5, vt5, idx5
        torch.cuda.empty_cache()

    if not args.no_published:
        log("bench: the reference's published shapes")
        try:
            result["published_shapes"] = published_bench(torch, dev)
        except Exception as e:  # reported, never fatal to the headline line
            result["published_shapes"] = {"error": repr(e)}
        torch.cuda.empty_cache()

    if args.calibrate_copy:
        x = torch.empty(128 * 1024 * 1024, device=dev, dtype=torch.bfloat16)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        result["copy_calibration_bytes"] = x.numel() * 2

    if not args.no_cpu:
        log("bench: CPU baseline (torch float32 restatement of the reference path)")
        result["cpu_baseline"] = cpu_baseline(p, dec_host, c5_cpu)
        try:
            model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo")
                         if l.startswith("model name"))
            result["cpu_baseline"]["cpu_model"] = model
        except Exception:
            pass

    print(json.dumps(compact(result)), flush=True)


def compact(result):
    """The JSON line with the nested figures rounded to 5 significant digits (value and
    ms_per_step in full), so that the line stays short."""
    def rnd(o):
        if isinstance(o, float):
            return float(f"{o:.5g}") if math.isfinite(o) and o != 0.0 else o
        if isinstance(o, dict):
            return {k: rnd(v) for k, v in o.items()}
        if isinstance(o, list):
            return [rnd(v) for v in o]
        return o
    return {k: (v if k in ("value", "ms_per_step") else rnd(v)) for k, v in result.items()}


if __name__ == "__main__":
    main()
