"""CPU tests of the C-ABI boundary: the library loads, exports every entry point the header
declares, and rejects invalid arguments with a status and a message (no GPU work is issued on
these paths)."""
import ctypes
import re
from pathlib import Path

import pytest

from ssa_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "ssa_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ssa_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_are_exported_and_bound():
    lib = _lib.lib()
    names = declared_functions()
    assert len(names) >= 14, names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in ssa_hip.h but not exported"
    assert sorted(_lib.exported_symbols()) == names


def test_abi_version_and_error_text():
    assert _lib.lib().ssa_abi_version() == _lib.ABI_VERSION
    with pytest.raises(_lib.SSAError, match="NULL"):
        _lib.call("ssa_sparse_attn_fwd", None, None, None, None, _lib.BF16, 1, 1, 1, 128, 64, 128,
                  _lib.i64_array([0] * 12), None, None, 1, 1.0, None, 0, None, 0, None)


def _status(name, *args):
    return getattr(_lib.lib(), name)(*args)


def test_invalid_arguments_are_rejected():
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: validation fails first
    st12 = _lib.i64_array([128 * 64, 128 * 64, 64] * 4)
    # head_dim 96 is not supported by the attention kernel
    rc = _status("ssa_sparse_attn_fwd", fake, fake, fake, fake, _lib.BF16, 1, 1, 1, 128, 96, 128,
                 st12, fake, fake, 1, 1.0, None, 0, None, 0, None)
    assert rc == _lib.SSA_ERR_UNSUPPORTED
    # block 96 is neither 64 nor a multiple of 128
    rc = _status("ssa_sparse_attn_fwd", fake, fake, fake, fake, _lib.BF16, 1, 1, 1, 128, 64, 96,
                 st12, fake, fake, 1, 1.0, None, 0, None, 0, None)
    assert rc == _lib.SSA_ERR_UNSUPPORTED
    # Hq not a multiple of Hkv
    rc = _status("ssa_sparse_attn_fwd", fake, fake, fake, fake, _lib.BF16, 1, 3, 2, 128, 64, 128,
                 st12, fake, fake, 1, 1.0, None, 0, None, 0, None)
    assert rc == _lib.SSA_ERR_INVALID
    # unknown dtype
    rc = _status("ssa_block_summary", fake, 7, 1, 1, 64, 64, 4096, 4096, 64, 64, 64, 0, fake, fake,
                 None, None)
    assert rc == _lib.SSA_ERR_UNSUPPORTED
    # QMEAN with a var output
    rc = _status("ssa_block_summary", fake, _lib.F32, 1, 1, 64, 64, 4096, 4096, 64, 64, 64,
                 _lib.STATS_QMEAN, fake, fake, None, None)
    assert rc == _lib.SSA_ERR_INVALID
    # route: W below the required width, then a too-small workspace
    rc = _status("ssa_route", fake, _lib.F32, fake, fake, None, 1, 1, 1, 16, 16, 64,
                 _lib.ROUTE_BUDGET, 4,
                 0.0, 1, 1.0, 0.0, 0, 1, fake, fake, 2, fake, 1 << 20, None)
    assert rc == _lib.SSA_ERR_INVALID
    rc = _status("ssa_route", fake, _lib.F32, fake, fake, None, 1, 1, 1, 16, 16, 64,
                 _lib.ROUTE_BUDGET, 4,
                 0.0, 1, 1.0, 0.0, 0, 1, fake, fake, 6, fake, 8, None)
    assert rc == _lib.SSA_ERR_WORKSPACE
    # decode: position outside the cache
    st12d = _lib.i64_array([64] * 12)
    rc = _status("ssa_decode_attend", fake, fake, fake, fake, _lib.BF16, 1, 1, 1, 1, 256, 64, 128,
                 256, st12d, fake, fake, 4, 1.0, fake, 1 << 20, None)
    assert rc == _lib.SSA_ERR_INVALID
    assert b"outside the cache" in _lib.lib().ssa_last_error()


def test_ivf_arguments_are_rejected():
    fake = ctypes.c_void_p(1 << 20)
    # index size grows with every dimension; zero for an empty shape
    assert _lib.query("ssa_ivf_index_size", 1, 1024, 32, 64) > 32 * 64 * 4 + 1024 * 4
    assert _lib.query("ssa_ivf_index_size", 0, 1024, 32, 64) == 0
    # d not a multiple of 32, nlist above nb, a small index buffer
    assert _status("ssa_ivf_build", fake, 1, 64, 48, 8, 10, fake, 1 << 30, None) == \
        _lib.SSA_ERR_UNSUPPORTED
    assert _status("ssa_ivf_build", fake, 1, 64, 64, 65, 10, fake, 1 << 30, None) == \
        _lib.SSA_ERR_UNSUPPORTED
    assert _status("ssa_ivf_build", fake, 1, 64, 64, 8, 10, fake, 64, None) == \
        _lib.SSA_ERR_WORKSPACE
    # route: search_k above 1024, the window above the LDS union, W too small
    args = lambda sk, top_c, local, W: (fake, fake, 1, 1, 4096, 64, 64, 4, sk, top_c, local,
                                        fake, fake, W, None)
    assert _status("ssa_ivf_route", *args(2048, 8, 1, 10)) == _lib.SSA_ERR_UNSUPPORTED
    assert _status("ssa_ivf_route", *args(1024, 1024, 2000, 4096)) == _lib.SSA_ERR_UNSUPPORTED
    assert _status("ssa_ivf_route", *args(16, 8, 1, 9)) == _lib.SSA_ERR_INVALID
    assert b"W=9" in _lib.lib().ssa_last_error()


def test_route_width():
    w = lambda *a: _lib.query("ssa_route_width", *a)  # noqa: E731
    # budget, top_c=64, local=2, 1024 blocks -> 64 + 3
    assert w(_lib.ROUTE_BUDGET, 1024, 1024, 64, 0.0, 2, 0, 1) == 67
    # budget_frac=1.0 over 16 blocks: last row keeps 15 + own
    assert w(_lib.ROUTE_BUDGET, 16, 16, -1, 1.0, 1, 0, 1) == 16
    # flat, tiny problem: capped at the block count
    assert w(_lib.ROUTE_FLAT, 4, 4, 8, 0.0, 1, 0, 1) == 4
    # query mode at position 1M-1, block 128: 64 routed + 2 local
    assert w(_lib.ROUTE_QUERY, 1, 8192, 64, 0.0, 1, 1048575, 128) == 66


def test_workspace_queries():
    # V^T (256-byte aligned), the fp16 copy of the bf16 keys (2 heads x 384 rows x 64), then the
    # fp32 key-norm maximum of every 64-key tile (2 heads x 6 tiles) and the per-(b, kv head) and
    # per-query-block flags, rounded up to 256 bytes
    assert _lib.query("ssa_sparse_attn_workspace_size", _lib.BF16, 1, 2, 300, 64, 128) == \
        2 * 64 * 384 * 2 + 2 * 384 * 64 * 2 + 256
    # fp16 keys are read directly: no copy
    assert _lib.query("ssa_sparse_attn_workspace_size", _lib.F16, 1, 2, 300, 64, 128) == \
        2 * 64 * 384 * 2 + 256
    # head dim 128 (exact path only): V^T and the flags
    assert _lib.query("ssa_sparse_attn_workspace_size", _lib.BF16, 1, 2, 300, 128, 128) == \
        2 * 128 * 384 * 2 + 256
    assert _lib.query("ssa_sparse_attn_workspace_size", _lib.F32, 1, 2, 300, 64, 128) == 0
    # per routed row: the score keys, then the certified scoring's error magnitude and largest
    # key per 64-candidate tile, and a deferred-row slot of the wave select; then its counters
    assert _lib.query("ssa_route_workspace_size", 1, 14, 1024, 1024) == \
        14 * 1024 * (1024 * 4 + 16 * 8 + 4) + 512
    assert _lib.query("ssa_decode_attend_workspace_size", 1, 14, 1, 66, 64) == 14 * 66 * 66 * 4


def test_cpu_tensors_raise():
    import torch
    from ssa_amd import ssa_kernel as K
    q = torch.randn(1, 1, 256, 64)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        K.ssa_flex(q, q, q)


def test_routing_projection_file_loads_without_pickle(tmp_path):
    """The reference's RoutingProjection.save format loads with weights_only=True."""
    import torch

    from ssa_amd import gemma_ssa as G
    path = tmp_path / "p.pt"
    wq, wk = torch.randn(64, 16), torch.randn(64, 16)
    torch.save({"W_q": wq, "W_k": wk, "meta": {"steps": 10, "name": "x"}}, path)
    p = G.load_projection(str(path), device="cpu")
    assert torch.equal(p.W_q, wq) and torch.equal(p.W_k, wk) and p.meta["steps"] == 10


def test_custom_op_fake_shapes():
    """The torch.library registrations (torch.compile's view of the kernels) give the shapes and
    dtypes of the real entry points; checked on meta tensors (their fake implementations)."""
    import torch
    import ssa_amd  # noqa: F401  (registers the ops)
    ops = torch.ops.ssa_amd
    m = dict(device="meta")
    q = torch.empty(1, 14, 1000, 64, dtype=torch.bfloat16, **m)
    k = torch.empty(1, 2, 1000, 64, dtype=torch.bfloat16, **m)
    assert ops.block_qmean(q, 128).shape == (1, 14, 8, 64)
    mu, var, m3 = ops.block_stats(k, 128, False, 1000, True)
    assert mu.shape == var.shape == m3.shape == (1, 2, 8, 64) and mu.dtype == torch.float32
    assert ops.block_stats(k, 128, False, -1, False)[2].numel() == 0
    qb = torch.empty(1, 14, 8, 64, dtype=torch.float32, **m)
    kv_num, kv_idx = ops.route(qb, mu, var, None, "budget", 4, 0.0, 2, 1.0, 0.0, 0, 1, 1)
    assert kv_num.shape == (1, 14, 8) and kv_idx.shape == (1, 14, 8, 7)
    assert kv_idx.dtype == torch.int32
    out = ops.sparse_attention(q, k, k, kv_num, kv_idx, 128, 0.125)
    assert out.shape == q.shape and out.dtype == q.dtype
    o2, lse = ops.sparse_attention_lse(q, k, k, kv_num, kv_idx, 128, 0.125)
    assert lse.shape == (1, 14, 1000) and lse.dtype == torch.float32
    qd = torch.empty(1, 14, 64, dtype=torch.bfloat16, **m)
    kc = torch.empty(1, 2, 4096, 64, dtype=torch.bfloat16, **m)
    kn = torch.empty(1, 2, 64, dtype=torch.bfloat16, **m)
    mus = torch.empty(1, 2, 32, 64, dtype=torch.float32, **m)
    num = torch.empty(1, 14, dtype=torch.int32, **m)
    idx = torch.empty(1, 14, 67, dtype=torch.int32, **m)
    o = ops.decode_step(qd, kn, kn, kc, kc, mus, mus, num, idx, None, 100, 128, 64, 0.0, 1, 1.0,
                        0.125)
    assert o.shape == (1, 14, 64)
