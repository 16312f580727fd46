"""eimoe_fused_moe_static, the entry point that allocates nothing, against eimoe_fused_moe.

Both are called through the C ABI with caller-owned outputs; the static one must give the same
bits (same kernels and launch shapes over its static scratch instead of the workspace), on two
calls in a row with the second smaller, and refuse a layer larger than its scratch before any
launch.
"""
import pytest
import torch

from easyinfra_amd import _lib, ops
from easyinfra_amd.workloads import SHAPES, make_inputs

pytestmark = pytest.mark.gpu


def _args(inp, dev, out, ids, w):
    s = inp.shape
    x, lg = inp.x.to(dev), inp.logits.to(dev)
    wgu, wd = inp.w_gate_up.to(dev), inp.w_down.to(dev)
    sg = inp.shared_gate_up.to(dev) if inp.shared_gate_up is not None else None
    sd = inp.shared_down.to(dev) if inp.shared_down is not None else None
    T, H = x.shape
    n_local, I2, _ = wgu.shape
    E = lg.shape[1]
    lo = inp.expert_range[0] if inp.expert_range is not None else 0
    Is = sd.shape[1] if sd is not None else 0
    flags = _lib.RENORMALIZE if s.renormalize else 0
    keep = (x, lg, wgu, wd, sg, sd)
    head = (x.data_ptr(), lg.data_ptr(), T, H, I2 // 2, E, s.top_k, wgu.data_ptr(), wd.data_ptr(), _lib.BF16,
            None, None, lo, n_local, ops._ptr(sg), ops._ptr(sd), Is, flags, out.data_ptr(), ops._dt(out))
    return keep, head, (ids.data_ptr(), w.data_ptr(), ops._stream(x)), (T, H, I2 // 2, E, s.top_k, n_local, Is,
                                                                        ops._dt(out), flags)


def _both(inp, dev, out_dtype):
    T, H = inp.x.shape
    k = inp.shape.top_k
    outs = []
    for static in (False, True):
        out = torch.full((T, H), float("nan"), dtype=out_dtype, device=dev)
        ids = torch.full((T, k), -7, dtype=torch.int32, device=dev)
        w = torch.full((T, k), float("nan"), dtype=torch.float32, device=dev)
        keep, head, tail, sizes = _args(inp, dev, out, ids, w)
        if static:
            _lib.call("eimoe_fused_moe_static", *head, *tail)
        else:
            need = int(_lib.lib().eimoe_fused_moe_workspace_bytes(*sizes))
            ws = torch.empty(need, dtype=torch.uint8, device=dev)
            _lib.call("eimoe_fused_moe", *head, ws.data_ptr(), need, *tail)
        torch.cuda.synchronize()
        outs.append((out.cpu(), ids.cpu(), w.cpu()))
    return outs


@pytest.mark.parametrize("name,T1,T2", [("deepseek-v2-lite", 300, 37), ("qwen3-30b-a3b-local32", 96, 5),
                                        ("mixtral-8x7b", 64, 1)])
def test_static_entry_point_matches_workspace_entry_point(dev, name, T1, T2):
    """Two calls in a row, the second with fewer tokens (the scratch keeps the first call's
    contents), each bit-identical to the workspace entry point."""
    for T, kw in ((T1, dict(hidden=256, inter=128)), (T2, dict(hidden=256, inter=128))):
        inp = make_inputs(SHAPES[name], T, device="cpu", **kw)
        (a, ia, wa), (b, ib, wb) = _both(inp, dev, torch.float32)
        assert torch.equal(ia, ib) and torch.equal(wa, wb)
        assert not torch.isnan(a).any()
        assert torch.equal(a, b)


def test_static_entry_point_at_mixtral_decode_shape(dev):
    """The real 64-token Mixtral-8x7B layer fits the 64 MiB scratch; then a 7-token call."""
    for T in (64, 7):
        inp = make_inputs(SHAPES["mixtral-8x7b"], T, device="cpu")
        (a, _, _), (b, _, _) = _both(inp, dev, torch.bfloat16)
        assert torch.equal(a, b)


def test_static_entry_point_refuses_a_layer_larger_than_its_scratch(dev):
    """The 8192-token Mixtral layer needs ~0.7 GB: refused with EIMOE_ERR_WORKSPACE, nothing launched."""
    cap = int(_lib.lib().eimoe_fused_moe_static_bytes())
    assert cap == 64 << 20
    need = int(_lib.lib().eimoe_fused_moe_workspace_bytes(8192, 4096, 14336, 8, 2, 8, 0, _lib.BF16,
                                                           _lib.RENORMALIZE))
    assert need > cap
    T, H, I, E = 8192, 4096, 14336, 8
    x = torch.zeros(T, H, dtype=torch.bfloat16, device=dev)
    lg = torch.zeros(T, E, dtype=torch.float32, device=dev)
    wgu = torch.zeros(1, dtype=torch.bfloat16, device=dev)   # never read: refused before any launch
    out = torch.full((T, H), 3.0, dtype=torch.bfloat16, device=dev)
    rc = _lib.lib().eimoe_fused_moe_static(x.data_ptr(), lg.data_ptr(), T, H, I, E, 2, wgu.data_ptr(),
                                           wgu.data_ptr(), _lib.BF16, None, None, 0, E, None, None, 0,
                                           _lib.RENORMALIZE, out.data_ptr(), _lib.BF16, None, None,
                                           ops._stream(x))
    assert rc == _lib.ERR_WORKSPACE
    assert "static" in _lib.last_error()
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
