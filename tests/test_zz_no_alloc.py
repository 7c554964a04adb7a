"""ssa_decode_step_static -- the allocation-free decode step (its scratch is the library's static
device array) -- against ssa_decode_step with a caller workspace, through the C ABI: two
decoders fed the same cache and steps must give bit-identical outputs and selections. The cases
run in a row, each smaller than the one before (the static array keeps the previous case's
contents), each crossing a block completion (a summary launch, the unfolded append); the second
takes the general four-launch step (more than 64 routed blocks), the others the fused one. The
first test captures a static step in a HIP graph -- the library's first look-up of its static
array's device address happens under capture -- and replays it."""
import numpy as np
import pytest
import torch

from ssa_amd import _lib
from ssa_amd import ivf_decode as D
from ssa_amd import workloads as WL

pytestmark = pytest.mark.gpu

CASES = [  # (Hq, Hkv, prefix, steps, block, top_c, dtype)
    (14, 2, 65536 + 100, 40, 128, 64, torch.bfloat16),
    (6, 2, 2000 + 30, 40, 16, 100, torch.bfloat16),
    (4, 1, 3000, 80, 64, 8, torch.float16),
]


def _decoders(cuda, Hq, Hkv, prefix, steps, block, top_c, dtype):
    rng = np.random.default_rng(prefix)
    total = prefix + steps
    k = WL.round_to(rng.standard_normal((1, Hkv, total, 64)).astype(np.float32), dtype)
    v = WL.round_to(rng.standard_normal((1, Hkv, total, 64)).astype(np.float32), dtype)
    q = WL.round_to(rng.standard_normal((steps, 1, Hq, 64)).astype(np.float32), dtype)
    kd, vd, qd = (WL.to_device(x, dtype, cuda) for x in (k, v, q))
    decs = [D.RoutedDecoder(1, Hq, Hkv, 64, total, block=block, top_c=top_c, local=1,
                            dtype=dtype, device=cuda, static_scratch=s) for s in (False, True)]
    for dec in decs:
        dec.prefill(kd[:, :, :prefix], vd[:, :, :prefix])
    return decs, kd, vd, qd


def test_static_step_captured_in_a_graph(cuda):
    """One static step captured with torch.cuda.graph (no allocation, no memset node: every
    buffer it touches exists before capture) and replayed three times, with eager steps of the
    workspace decoder and host synchronisations between the replays: each replay rewrites the same
    position, so its output, selection and caches equal the workspace decoder's eager step at that
    position bit for bit."""
    Hq, Hkv, prefix, block, top_c, dtype = 14, 2, 8192 + 60, 128, 64, torch.bfloat16
    print("graph-captured static decode step", flush=True)
    decs, kd, vd, qd = _decoders(cuda, Hq, Hkv, prefix, 4, block, top_c, dtype)
    ref_dec, st_dec = decs
    qs, ks, vs = qd[0].clone(), kd[:, :, prefix].contiguous(), vd[:, :, prefix].contiguous()
    out_s = torch.empty(1, Hq, 64, device=cuda, dtype=dtype)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st_dec.step(qs, ks, vs, out=out_s)
    st_dec.pos = prefix  # capture ran no kernel: the graph performs the step at `prefix`
    out_r = ref_dec.step(qs, ks, vs)
    torch.cuda.synchronize()
    for rep in range(3):
        out_s.zero_()
        st_dec.kv_idx.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_s, out_r), rep
        assert torch.equal(st_dec.kv_num, ref_dec.kv_num), rep
        assert torch.equal(st_dec.kv_idx, ref_dec.kv_idx), rep
        assert torch.equal(st_dec.kcache, ref_dec.kcache), rep
        # the program's own eager work between replays
        torch.empty(1 << 20, device=cuda).normal_().sum().item()


@pytest.mark.parametrize("case", CASES)
def test_static_scratch_step_equals_workspace_step(cuda, case):
    Hq, Hkv, prefix, steps, block, top_c, dtype = case
    print(f"static decode case {case}", flush=True)
    decs, kd, vd, qd = _decoders(cuda, Hq, Hkv, prefix, steps, block, top_c, dtype)
    assert decs[1].workspace is None
    outs = [torch.empty(1, Hq, 64, device=cuda, dtype=dtype) for _ in decs]
    completed = 0
    for t in range(steps):
        pos = prefix + t
        completed += (pos + 1) % block == 0
        for dec, o in zip(decs, outs):
            dec.step(qd[t], kd[:, :, pos].contiguous(), vd[:, :, pos].contiguous(), out=o)
        assert torch.equal(outs[0], outs[1]), t
        assert torch.equal(decs[0].kv_num, decs[1].kv_num), t
        assert torch.equal(decs[0].kv_idx, decs[1].kv_idx), t
    assert completed >= 1
    assert torch.equal(decs[0].kcache, decs[1].kcache)
    assert torch.equal(decs[0].mu, decs[1].mu) and torch.equal(decs[0].var, decs[1].var)
    assert torch.isfinite(outs[1].float()).all()


def test_static_scratch_rejects_oversized_steps(cuda):
    """A step whose scratch exceeds the static array is refused with SSA_ERR_WORKSPACE (checked
    on the host before anything is launched), by the C ABI and by RoutedDecoder."""
    x = torch.zeros(1, 1, 64, device=cuda, dtype=torch.bfloat16)
    i32 = torch.zeros(1, 72, device=cuda, dtype=torch.int32)
    strides = _lib.i64_array([64, 64, 64, 64, 64, 64, 64, 64, 64, 64, 64, 64, 64, 64])
    cap = 1 << 31  # B*Hq*(cap/block)*4 bytes of score keys alone exceed the array
    with pytest.raises(_lib.SSAError) as e:
        _lib.call("ssa_decode_step_static", x.data_ptr(), x.data_ptr(), x.data_ptr(),
                  x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), _lib.BF16,
                  1, 14, 2, cap, 64, 64, 0, strides, 64, 0.0, 1, 1.0, 0.125, i32.data_ptr(),
                  i32.data_ptr(), 72, _lib.stream_of(x))
    assert e.value.status == _lib.SSA_ERR_WORKSPACE
    with pytest.raises(ValueError):
        D.RoutedDecoder(1, 14, 2, 64, 1 << 26, block=64, top_c=64, device=cuda,
                        static_scratch=True)
