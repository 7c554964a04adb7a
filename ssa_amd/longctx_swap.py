"""Real-model prefill timing and smoke gate of the attention swap (drop-in for
ssa/longctx_swap.py:32-79,153-162) on the HIP path.

    python -m ssa_amd.longctx_swap --lengths 32768,131072 --budgets 1.0,0.25,0.12,0.06

`load` builds the Qwen2.5-0.5B architecture (24 decoder layers, hidden 896, 14 query / 2 key
heads, d 64, vocab 151936, bf16) from a local checkpoint directory when one is given, otherwise
with seeded random weights (no checkpoint can be fetched by name here). Lengths above the
native 32768-token window run under YaRN x4 for the dense and the routed model alike
(ssa/longctx_swap.py:36-43). `prefill_ms` is the reference's measure: median wall-clock of
model(ids, logits_to_keep=1) over `reps` runs after `warmup` runs, plus peak memory. The smoke
gate requires the full-budget swap to reproduce the dense LM loss within 5e-2
(ssa/longctx_swap.py:153-162); with random weights the loss is taken on seeded random tokens.
"""
from __future__ import annotations

import argparse
import json
import os
import time

import torch

from . import gemma_ssa as G

QWEN05B = dict(vocab_size=151936, hidden_size=896, intermediate_size=4864, num_hidden_layers=24,
               num_attention_heads=14, num_key_value_heads=2, tie_word_embeddings=True,
               rms_norm_eps=1e-6)


def load(path: str | None = None, yarn: bool = False, device="cuda", seed: int = 0,
         layers: int | None = None):
    """(model, source): the Qwen2.5-0.5B architecture in bf16 on `device`, eval mode, attention
    "sdpa"; weights from `path` (a local transformers checkpoint directory) or seeded random."""
    from transformers import AutoConfig, AutoModelForCausalLM, Qwen2Config, Qwen2ForCausalLM
    rope = {"rope_type": "default", "rope_theta": 1e6}
    if yarn:  # the reference extends the 32768-token window x4 with YaRN, keeping the base
        rope = {"rope_type": "yarn", "factor": 4.0, "original_max_position_embeddings": 32768,
                "rope_theta": 1e6}
    max_pos = 131072 if yarn else 32768
    if path and os.path.isdir(path):
        cfg = AutoConfig.from_pretrained(path, local_files_only=True)
        if yarn:
            cfg.rope_parameters = rope
            cfg.max_position_embeddings = max_pos
        cfg._attn_implementation = "sdpa"
        model = AutoModelForCausalLM.from_pretrained(path, config=cfg, dtype=torch.bfloat16,
                                                     local_files_only=True)
        source = path
    else:
        kw = dict(QWEN05B)
        if layers is not None:
            kw["num_hidden_layers"] = int(layers)
        cfg = Qwen2Config(**kw, rope_parameters=rope, max_position_embeddings=max_pos,
                          attn_implementation="sdpa")
        torch.manual_seed(seed)
        model = Qwen2ForCausalLM(cfg)
        source = f"random weights (seed {seed})"
    return model.to(device=device, dtype=torch.bfloat16).eval(), source


def prefill_ms(model, ids, warmup: int = 2, reps: int = 3):
    """Median prefill wall-clock in ms and peak allocated memory in GB
    (ssa/longctx_swap.py:61-79): logits_to_keep=1 keeps the vocabulary matmul out of the timing."""
    torch.cuda.reset_peak_memory_stats()
    with torch.no_grad():
        for _ in range(warmup):
            model(ids, logits_to_keep=1)
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            model(ids, logits_to_keep=1)
            torch.cuda.synchronize()
            ts.append((time.perf_counter() - t0) * 1e3)
    ts.sort()
    return ts[len(ts) // 2], torch.cuda.max_memory_allocated() / 1e9


def lm_loss(model, ids) -> float:
    with torch.no_grad():
        return float(model(ids, labels=ids).loss.item())


def use_dense(model):
    """Back to the stock attention (torch SDPA) after install_ssa."""
    model.config._attn_implementation = "sdpa"


def smoke_gate(model, ids, block: int = 128, beta: float = 2.0, tol: float = 5e-2):
    """(dense loss, full-budget swap loss, passed): ssa/longctx_swap.py:153-162."""
    use_dense(model)
    base = lm_loss(model, ids)
    G.install_ssa(model, block=block, budget_frac=1.0, beta=beta, impl="hip")
    gated = lm_loss(model, ids)
    return base, gated, abs(gated - base) < tol


def run(lengths, budgets, block=128, beta=2.0, path=None, warmup=2, reps=3, seed=0, layers=None,
        device="cuda", log=print):
    """Dense rows, the smoke gate, then the budget grid (ssa/longctx_swap.py:136-179);
    returns the rows."""
    yarn = any(n > 32768 for n in lengths)
    model, source = load(path, yarn=yarn, device=device, seed=seed, layers=layers)
    g = torch.Generator().manual_seed(seed)
    rows = []
    for n in sorted(lengths):
        ids = torch.randint(0, model.config.vocab_size, (1, n), generator=g).to(device)
        use_dense(model)
        ms, mem = prefill_ms(model, ids, warmup, reps)
        rows.append({"impl": "dense", "n": n, "budget": 1.0, "prefill_ms": ms, "peak_mem_gb": mem})
        log(f"  dense n={n}: {ms:.1f} ms, {mem:.2f} GB")
    gate_ids = torch.randint(0, model.config.vocab_size, (1, 512), generator=g).to(device)
    base, gated, ok = smoke_gate(model, gate_ids, block=block, beta=beta)
    log(f"  [smoke] dense={base:.4f} swap@1.0={gated:.4f} {'PASS' if ok else 'FAIL'}")
    gate = {"dense_loss": base, "swap_loss": gated, "passed": ok}
    if not ok:
        return {"source": source, "rope": "yarn4" if yarn else "native", "smoke": gate,
                "rows": rows}
    for n in sorted(lengths):
        ids = torch.randint(0, model.config.vocab_size, (1, n), generator=g).to(device)
        dense_ms = next(r["prefill_ms"] for r in rows if r["impl"] == "dense" and r["n"] == n)
        for b in budgets:
            G.install_ssa(model, block=block, budget_frac=b, beta=beta, impl="hip")
            ms, mem = prefill_ms(model, ids, warmup, reps)
            rows.append({"impl": "hip", "n": n, "budget": b, "prefill_ms": ms, "peak_mem_gb": mem,
                         "speedup_vs_dense": dense_ms / ms})
            log(f"  hip n={n} budget={b}: {ms:.1f} ms ({dense_ms / ms:.2f}x), {mem:.2f} GB")
    use_dense(model)
    return {"source": source, "rope": "yarn4" if yarn else "native", "smoke": gate, "rows": rows}


def main():
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--model-path", default=None, help="local Qwen2.5-0.5B checkpoint directory")
    ap.add_argument("--lengths", default="8192,16384,32768")
    ap.add_argument("--budgets", default="1.0,0.25,0.12,0.06")
    ap.add_argument("--block", type=int, default=128)
    ap.add_argument("--beta", type=float, default=2.0)
    ap.add_argument("--out", default=None)
    args = ap.parse_args()
    res = run([int(x) for x in args.lengths.split(",")],
              [float(x) for x in args.budgets.split(",")], block=args.block, beta=args.beta,
              path=args.model_path)
    if args.out:
        with open(args.out, "w") as f:
            json.dump(res, f, indent=2)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
