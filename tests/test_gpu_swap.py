"""GPU parity tests of the trainable attention swap (ssa_amd.ssa_swap, drop-in for
ssa/ssa_swap.py:32-63): per-query routing through the HIP router (SSA_ROUTE_STARTED), the
block-sparse forward and its backward (ssa_masked_attn_fwd / _bwd), against the float64 oracle
and the reference's own float32 forward + autograd gradients (tests/golden/swap_masked_*.npz).

Bars: selections bit-exact against the oracle; outputs and gradients within 1e-5 (fp32) or
2e-2 (bf16/fp16) max-abs of the oracle (gradients of bf16/fp16 inputs are compared relative to
their largest magnitude, at the same 2e-2)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ssa_oracle as O
from ssa_amd import ssa_swap as S
from ssa_amd import workloads as WL
from tests import golden_util as GU

pytestmark = pytest.mark.gpu


def np_of(t):
    return t.detach().float().cpu().numpy()


def run_masked(q, k, v, g, block, top_c, local, dtype, cuda):
    tq, tk, tv = (WL.to_device(x, dtype, cuda).requires_grad_(True) for x in (q, k, v))
    out = S.ssa_masked(tq, tk, tv, block, top_c, local)
    out.backward(WL.to_device(g, dtype, cuda))
    torch.cuda.synchronize()
    return out, tq.grad, tk.grad, tv.grad


def assert_selection_equals_oracle(q, k, block, top_c, local, dtype, cuda):
    tq, tk = (WL.to_device(x, dtype, cuda) for x in (q, k))
    kv_num, kv_idx = S.route_masked(tq, tk, block, top_c, local)
    sel = O.masked_route(q, k, block, top_c, local)
    got = GU.row_sets(kv_num.cpu().numpy(), kv_idx.cpu().numpy())
    assert got == [frozenset(x) for x in sel.ravel()]
    return sel


@pytest.mark.parametrize("name", list(GU.MASKED_CASES))
def test_ssa_masked_matches_reference(cuda, name):
    """fp32: selection == oracle, and out / dq / dk / dv within 1e-5 of the reference's own
    forward and autograd gradients."""
    seed, (b, h, n, d), block, top_c, local = GU.MASKED_CASES[name]
    q, k, v, g = GU.masked_inputs(seed, b, h, n, d)
    ref = GU.load(name)
    assert GU.sha(q, k, v, g) == str(ref["inputs_sha256"])
    assert_selection_equals_oracle(q, k, block, top_c, local, torch.float32, cuda)
    res = run_masked(q, k, v, g, block, top_c, local, torch.float32, cuda)
    for got, key in zip(res, ("out", "dq", "dk", "dv")):
        assert np.abs(np_of(got) - ref[key]).max() < 1e-5, key


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 4, 2, 333, 64, 32, 2, 1), (2, 2, 1, 130, 128, 16, 4, 2),
                                   (1, 2, 2, 17, 64, 16, 1, 0), (1, 2, 2, 1, 64, 16, 3, 1)])
def test_ssa_masked_matches_oracle(cuda, dtype, shape):
    """GQA, head_dim 128, ragged tails, a single query row: forward and gradients against the
    float64 oracle on the dtype-rounded inputs."""
    b, hq, hkv, n, d, block, top_c, local = shape
    rng = np.random.default_rng(hash(shape) % 2**32)
    q = WL.round_to(rng.standard_normal((b, hq, n, d)).astype(np.float32), dtype)
    k, v = (WL.round_to(rng.standard_normal((b, hkv, n, d)).astype(np.float32), dtype)
            for _ in range(2))
    g = WL.round_to(rng.standard_normal((b, hq, n, d)).astype(np.float32), dtype)
    sel = assert_selection_equals_oracle(q, k, block, top_c, local, dtype, cuda)
    out, dq, dk, dv = run_masked(q, k, v, g, block, top_c, local, dtype, cuda)
    oout, _ = O.masked_forward(q, k, v, sel, block)
    odq, odk, odv = O.masked_grads(q, k, v, sel, g, block)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert np.abs(np_of(out) - oout).max() < tol
    for got, want, nm in ((dq, odq, "dq"), (dk, odk, "dk"), (dv, odv, "dv")):
        scale = 1.0 if dtype == torch.float32 else max(1.0, np.abs(want).max())
        assert np.abs(np_of(got) - want).max() < tol * scale, nm


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_bwd_fresh_workspace_equals_reused_masks(cuda, dtype):
    """ssa_masked_attn_bwd on a fresh workspace (flags 0: it builds the row masks itself), with
    fp32 gradients, equals the autograd backward, which reuses the forward's masks and writes
    the gradients in the input type."""
    from ssa_amd import _lib
    rng = np.random.default_rng(23)
    B, H, n, d, block = 1, 2, 200, 64, 32
    q, k, v, g = (rng.standard_normal((B, H, n, d)).astype(np.float32) for _ in range(4))
    out, dq, dk, dv = run_masked(q, k, v, g, block, 2, 1, dtype, cuda)
    tq, tk, tv, tg = (WL.to_device(x, dtype, cuda) for x in (q, k, v, g))
    kv_num, kv_idx = S.route_masked(tq, tk, block, 2, 1)
    W = kv_idx.shape[-1]
    o2, lse = torch.empty_like(tq), torch.empty(B, H, n, device=cuda, dtype=torch.float32)
    wsb = int(_lib.query("ssa_masked_attn_workspace_size", B, H, n, W, d, block))
    strides = S._strides(tq, tk, tv, o2)
    dt = _lib.dtype_code(dtype)
    ws = torch.empty(wsb, device=cuda, dtype=torch.uint8)
    _lib.call("ssa_masked_attn_fwd", tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), o2.data_ptr(),
              lse.data_ptr(), dt, B, H, H, n, d, block, strides, kv_num.data_ptr(),
              kv_idx.data_ptr(), W, d ** -0.5, ws.data_ptr(), wsb, _lib.stream_of(tq))
    grads = [torch.empty(B, H, n, d, device=cuda, dtype=torch.float32) for _ in range(3)]
    fresh = torch.empty(wsb, device=cuda, dtype=torch.uint8)
    _lib.call("ssa_masked_attn_bwd", tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), o2.data_ptr(),
              tg.data_ptr(), lse.data_ptr(), *(x.data_ptr() for x in grads), dt, _lib.F32, 0,
              B, H, H, n, d, block, strides, kv_num.data_ptr(), kv_idx.data_ptr(), W, d ** -0.5,
              fresh.data_ptr(), wsb, _lib.stream_of(tq))
    torch.cuda.synchronize()
    assert torch.equal(o2, out)
    for got, ref in zip(grads, (dq, dk, dv)):
        assert torch.equal(got.to(dtype), ref)


def test_ssa_masked_strided_views(cuda):
    """GPT-2 hands SDPA q/k/v as head-transposed views of one fused projection: the same
    results as on contiguous copies, without a copy of the inputs."""
    rng = np.random.default_rng(21)
    b, h, n, d = 2, 4, 200, 64
    qkv = torch.from_numpy(rng.standard_normal((b, n, 3 * h * d)).astype(np.float32)).to(cuda)
    q, k, v = (t.view(b, n, h, d).transpose(1, 2) for t in qkv.split(h * d, dim=2))
    assert not q.is_contiguous()
    out = S.ssa_masked(q, k, v, 32, 2, 1)
    ref = S.ssa_masked(q.contiguous(), k.contiguous(), v.contiguous(), 32, 2, 1)
    assert torch.equal(out, ref)


def test_patched_sdpa_switch(cuda):
    """install() replaces F.scaled_dot_product_attention: with _SSA["on"] it is ssa_masked with
    the switch's block / top_c / local, off it is torch's own; uninstall() restores it."""
    rng = np.random.default_rng(22)
    q, k, v = (torch.from_numpy(rng.standard_normal((1, 2, 150, 64)).astype(np.float32)).to(cuda)
               for _ in range(3))
    saved = dict(S._SSA)
    try:
        S.install()
        assert F.scaled_dot_product_attention is S._patched_sdpa
        S._SSA.update(on=False)
        dense = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        assert torch.equal(dense, S._orig_sdpa(q, k, v, is_causal=True))
        S._SSA.update(on=True, block=32, top_c=2, local=1)
        sparse = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        assert torch.equal(sparse, S.ssa_masked(q, k, v, 32, 2, 1))
        assert (sparse - dense).abs().max().item() > 1e-3
        S._SSA.update(top_c=99)  # every begun block kept: token-causal dense attention
        assert (F.scaled_dot_product_attention(q, k, v) - dense).abs().max().item() < 1e-5
    finally:
        S.uninstall()
        S._SSA.clear()
        S._SSA.update(saved)
    assert F.scaled_dot_product_attention is S._orig_sdpa


def test_gpt2_swap_trains(cuda):
    """The reference's swap on a transformers GPT-2 (random weights, 2 layers; no checkpoint
    can be fetched here): at top_c >= blocks the swapped model's loss and attention-weight
    gradients equal SDPA's; at top_c=4 / local=2 the loss differs and one AdamW step through
    the sparse attention lowers it on the batch."""
    from transformers import GPT2Config, GPT2LMHeadModel
    cfg = GPT2Config(vocab_size=512, n_positions=1024, n_embd=256, n_layer=2, n_head=4,
                     attn_implementation="sdpa")
    torch.manual_seed(0)
    model = GPT2LMHeadModel(cfg).to(cuda).train()
    model.config.attn_pdrop = model.config.resid_pdrop = model.config.embd_pdrop = 0.0
    for m in model.modules():
        if isinstance(m, torch.nn.Dropout):
            m.p = 0.0
    ids = torch.randint(0, 512, (2, 1024), device=cuda)
    w = model.transformer.h[0].attn.c_attn.weight

    def loss_and_grad():
        model.zero_grad(set_to_none=True)
        loss = model(ids, labels=ids).loss
        loss.backward()
        return loss.item(), w.grad.detach().clone()

    saved = dict(S._SSA)
    try:
        S.install()
        S._SSA.update(on=False)
        dense_loss, dense_grad = loss_and_grad()
        S._SSA.update(on=True, block=64, top_c=99, local=2)
        full_loss, full_grad = loss_and_grad()
        assert abs(full_loss - dense_loss) < 1e-4
        assert (full_grad - dense_grad).abs().max().item() < 1e-4 * max(1.0, dense_grad.abs().max().item())
        S._SSA.update(top_c=4)
        sparse_loss, sparse_grad = loss_and_grad()
        assert abs(sparse_loss - dense_loss) > 1e-5 and torch.isfinite(sparse_grad).all()
        opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
        opt.step()
        with torch.no_grad():
            after = model(ids, labels=ids).loss.item()
        assert after < sparse_loss
    finally:
        S.uninstall()
        S._SSA.clear()
        S._SSA.update(saved)


def test_longctx_prefill_timing_and_smoke_gate(cuda):
    """ssa_amd.longctx_swap on a 2-layer Qwen2.5-0.5B-shaped model (random weights): the dense
    row, the smoke gate (full-budget swap reproduces the dense loss within 5e-2) and the budget
    rows run end to end (ssa/longctx_swap.py:61-79,136-179)."""
    from ssa_amd import gemma_ssa as G
    from ssa_amd import longctx_swap as L
    res = L.run([2048], [1.0, 0.25], layers=2, warmup=1, reps=1, log=lambda *a: None)
    assert res["smoke"]["passed"], res["smoke"]
    impls = [(r["impl"], r["budget"]) for r in res["rows"]]
    assert impls == [("dense", 1.0), ("hip", 1.0), ("hip", 0.25)]
    assert all(r["prefill_ms"] > 0 for r in res["rows"])
    G.CFG.__dict__.update(G.SSAConfig().__dict__)
