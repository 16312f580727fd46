"""The fused layer and the MoE prologue under HIP graph capture.

A serving loop captures the layer once and replays it with new contents in the same
input buffers.  Each replay must equal an eager call on the same inputs bit for bit (the
layer is deterministic), with eager work and synchronisations between the replays.  The
DeepSeek-V2-Lite case forks its shared experts onto a second stream and joins it back,
which the capture has to follow; the W8A8 case adds the activation quantisation kernels.
"""
import pytest
import torch

from easyinfra_amd import ops
from easyinfra_amd.workloads import SHAPES, make_inputs

pytestmark = pytest.mark.gpu


def _kwargs(inp, dev):
    s = inp.shape
    kw = dict(renormalize=s.renormalize, expert_range=inp.expert_range)
    if inp.shared_gate_up is not None:
        kw.update(shared_gate_up=inp.shared_gate_up.to(dev), shared_down=inp.shared_down.to(dev))
    return kw


# 4096 Mixtral tokens (8192 routed pairs) take the many-workgroup align inside the graph.
@pytest.mark.parametrize("name,T,w8a8", [("deepseek-v2-lite", 48, False), ("mixtral-8x7b", 96, False),
                                         ("qwen3-30b-a3b-local32", 40, False), ("mixtral-8x7b", 64, True),
                                         ("mixtral-8x7b", 4096, False)])
def test_fused_moe_graph_replays_match_eager(dev, name, T, w8a8):
    shape = SHAPES[name]
    inp = make_inputs(shape, T, device="cpu", hidden=256, inter=128)
    kw = _kwargs(inp, dev)
    wgu, wd = inp.w_gate_up.to(torch.bfloat16).to(dev), inp.w_down.to(torch.bfloat16).to(dev)
    if w8a8:
        qgu, sgu = ops.quantize_weights_fp8(wgu)
        qd, sd = ops.quantize_weights_fp8(wd)
        wgu, wd = qgu, qd
        kw.update(w_scales=(sgu, sd), w8a8=True)
    g = torch.Generator().manual_seed(T)
    xs = [inp.x.to(torch.bfloat16)] + [(torch.randn(inp.x.shape, generator=g) * (1 + j)).to(torch.bfloat16)
                                       for j in range(2)]
    lgs = [inp.logits.float()] + [torch.randn(inp.logits.shape, generator=g) * 2 for _ in range(2)]
    xs = [x.to(dev) for x in xs]
    lgs = [lg.to(dev) for lg in lgs]
    k = shape.top_k

    eager = [ops.fused_moe(x, lg, k, wgu, wd, **kw) for x, lg in zip(xs, lgs)]
    torch.cuda.synchronize()

    x_s, lg_s = xs[0].clone(), lgs[0].clone()
    n_local = wgu.shape[0]
    Is = kw["shared_down"].shape[1] if "shared_down" in kw else 0
    need = ops.fused_moe_workspace_bytes(T, x_s.shape[1], wd.shape[2], shape.n_experts, k, n_local, Is,
                                         flags=4 if w8a8 else 0)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # warm-up on the capture stream, as torch requires
        ops.fused_moe(x_s, lg_s, k, wgu, wd, workspace=ws, **kw)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_s = ops.fused_moe(x_s, lg_s, k, wgu, wd, workspace=ws, **kw)

    for j in (1, 0, 2, 1):
        x_s.copy_(xs[j])
        lg_s.copy_(lgs[j])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_s, eager[j]), f"replay with inputs {j} differs from the eager call"
        # eager work between replays (its own workspace), then the next replay
        again = ops.fused_moe(xs[2 - j // 2], lgs[2 - j // 2], k, wgu, wd, **kw)
        torch.cuda.synchronize()
        assert torch.equal(again, eager[2 - j // 2])


# The prologue's router GEMM path (K-split planes and their sum, the segment offsets written
# by the norm kernel) and its one-pass path, replayed with new inputs.
@pytest.mark.parametrize("T,H,E,lbf16", [(512, 7168, 256, False), (300, 4096, 8, True)])
def test_moe_prologue_graph_replays_match_eager(dev, T, H, E, lbf16):
    g = torch.Generator().manual_seed(T + E)
    hs = [(torch.randn(T, H, generator=g) * (1 + j)).to(torch.bfloat16).to(dev) for j in range(3)]
    rs = [torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev) for _ in range(3)]
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    gw = (0.05 * torch.randn(E, H, generator=g)).to(torch.bfloat16).to(dev)
    eager = [ops.moe_prologue(h, r, w, 1e-6, gw, lbf16) for h, r in zip(hs, rs)]
    torch.cuda.synchronize()
    h_s, r_s = hs[0].clone(), rs[0].clone()
    need = ops.moe_prologue_workspace_bytes(T, H, E)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.moe_prologue(h_s, r_s, w, 1e-6, gw, lbf16, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_s = ops.moe_prologue(h_s, r_s, w, 1e-6, gw, lbf16, workspace=ws)
    for j in (2, 0, 1):
        h_s.copy_(hs[j])
        r_s.copy_(rs[j])
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(out_s, eager[j]):
            assert torch.equal(got, want), f"replay with inputs {j} differs from the eager call"
        again = ops.moe_prologue(hs[2 - j], rs[2 - j], w, 1e-6, gw, lbf16)
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(again, eager[2 - j]))
