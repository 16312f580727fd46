"""fp8 paths on the GPU.

W8A8 (fp8 activations and weights on the fp8 MFMA): each GEMM is compared with the
oracle on the same quantised operands (tight: only fp32 accumulation order differs),
and the layer with the oracle's W8A8 forward (1e-2).  Against the bf16 fp32
reference the W8A8 layer carries e4m3 rounding of both operands of both GEMMs:
6.5 % rel-L2 at the Mixtral shape, which the stated 5e-2 cannot hold (rounding x
and W_gate_up alone exceeds it, tests/test_oracle.py pins that on the CPU), so the
W8A8 layer is held to the measured e4m3 floor with margin (7.5e-2).  The W8A16 layer
(fp8 weights, bf16 activations) meets 5e-2.
"""
import numpy as np
import pytest
import torch

import oracle
from easyinfra_amd import ops
from easyinfra_amd.workloads import SHAPES, make_inputs

pytestmark = pytest.mark.gpu


def cpu(t):
    return t.detach().cpu()


def _segments(counts):
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return off, torch.as_tensor(off)


# tile 5 = the weight-streaming kernel (fp8 operands on the 16x16x128 fp8 MFMA); H=1024
# reaches its 4-wave K split with a 2-deep register ring, H=256 the unsplit ring.
@pytest.mark.parametrize("tile,H", [(1, 256), (2, 256), (3, 256), (4, 256), (5, 256), (5, 1024), (5, 4096)])
def test_w8a8_gate_up_matches_oracle(dev, tile, H):
    g = torch.Generator().manual_seed(tile + H)
    I, T = 256, 50
    counts = [0, 37, 300, 5]
    E = len(counts)
    off, off_t = _segments(counts)
    rows = int(off[-1])
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    a_rows = torch.randint(0, T, (rows,), generator=g, dtype=torch.int32)
    w = torch.randn(E, 2 * I, H, generator=g) * 0.02
    qw, sw = oracle.quantize_weights_fp8(w)
    xq, sx = oracle.quantize_rows_fp8(x)
    h = ops.gemm_gate_up_silu_w8a8(xq.to(dev), sx.to(dev), qw.to(dev), sw.to(dev), off_t.to(dev), rows,
                                   a_rows=a_rows.to(dev), tile=tile)
    h = cpu(h).float()
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b == a:
            continue
        tok = a_rows[a:b].long()
        gu = (xq[tok].float() @ qw[e].float().T) * sx[tok][:, None] * sw[e][None, :]
        ref = oracle.silu(gu[:, :I]) * gu[:, I:]
        torch.testing.assert_close(h[a:b], ref, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("tile,k_split", [(1, 1), (2, 1), (3, 2), (4, 1), (5, 1), (5, 2)])
def test_w8a8_down_matches_oracle(dev, tile, k_split):
    g = torch.Generator().manual_seed(10 + tile)
    H, I = 256, 512
    counts = [3, 0, 260, 41]
    E = len(counts)
    off, off_t = _segments(counts)
    rows = int(off[-1])
    h = torch.randn(rows, I, generator=g) * 0.5
    hq, sh = oracle.quantize_rows_fp8(h)
    w = torch.randn(E, H, I, generator=g) * 0.02
    qw, sw = oracle.quantize_weights_fp8(w)
    y = ops.gemm_down_w8a8(hq.to(dev), sh.to(dev), qw.to(dev), sw.to(dev), off_t.to(dev), rows, k_split=k_split,
                           tile=tile)
    y = cpu(y).sum(0)
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        ref = (hq[a:b].float() @ qw[e].float().T) * sh[a:b][:, None] * sw[e][None, :]
        torch.testing.assert_close(y[a:b], ref, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("name,T", [("mixtral-8x7b-fp8", 96), ("mixtral-8x7b-fp8", 7), ("qwen3-30b-a3b-local32", 64)])
def test_w8a8_layer(dev, name, T):
    inp = make_inputs(SHAPES[name], T, device="cpu", hidden=256, inter=256)
    s = inp.shape
    qgu, sgu = oracle.quantize_weights_fp8(inp.w_gate_up.float())
    qd, sd = oracle.quantize_weights_fp8(inp.w_down.float())
    out = ops.fused_moe(inp.x.to(dev), inp.logits.to(dev), s.top_k, qgu.to(dev), qd.to(dev),
                        renormalize=s.renormalize, expert_range=inp.expert_range,
                        w_scales=(sgu.to(dev), sd.to(dev)), out_dtype=torch.float32, w8a8=True)
    got = cpu(out)
    ref8 = oracle.moe_forward_fp8(inp.x, inp.logits, s.top_k, qgu, sgu, qd, sd, s.renormalize, mode="w8a8",
                                  expert_range=inp.expert_range)
    ref = oracle.moe_forward(inp.x, inp.logits, s.top_k, inp.w_gate_up, inp.w_down, s.renormalize,
                             expert_range=inp.expert_range)
    # h is quantised from its bf16 copy on both sides; fp32 accumulation order can still flip a
    # rare bf16 / e4m3 rounding, hence a looser bound than the GEMM checks above.
    assert oracle.rel_l2(got, ref8) <= 1e-2
    print(f"{name} T={T}: W8A8 vs W8A8-oracle {oracle.rel_l2(got, ref8):.3e}, vs bf16-ref {oracle.rel_l2(got, ref):.3e}")
    assert oracle.rel_l2(got, ref) <= 7.5e-2


def test_w8a16_layer_meets_fp8_tolerance(dev):
    inp = make_inputs(SHAPES["mixtral-8x7b-fp8"], 96, device="cpu", hidden=256, inter=256)
    qgu, sgu = oracle.quantize_weights_fp8(inp.w_gate_up.float())
    qd, sd = oracle.quantize_weights_fp8(inp.w_down.float())
    out = ops.fused_moe(inp.x.to(dev), inp.logits.to(dev), 2, qgu.to(dev), qd.to(dev),
                        w_scales=(sgu.to(dev), sd.to(dev)), out_dtype=torch.float32)
    ref = oracle.moe_forward(inp.x, inp.logits, 2, inp.w_gate_up, inp.w_down, True)
    ref16 = oracle.moe_forward_fp8(inp.x, inp.logits, 2, qgu, sgu, qd, sd, True, mode="w8a16")
    assert oracle.rel_l2(cpu(out), ref16) <= 1e-2
    assert oracle.rel_l2(cpu(out), ref) <= 5e-2


@pytest.mark.slow
@pytest.mark.parametrize("T", [1, 8, 64, 8192])
def test_fp8_mixtral_real_shape(dev, T):
    """Mixtral-8x7B with fp8-e4m3 weights (per-channel absmax/448), every row, against the bf16
    fp32 reference and against the oracle's own fp8 forward of the same mode (1 token: the
    streaming kernels; 8: W8A8 on the 16x64 tiles with non-temporal weight DMA; 64 and 8192: the
    32x128 and 256x256 tiles)."""
    import json
    inp = make_inputs(SHAPES["mixtral-8x7b-fp8"], T, device=dev)
    qgu, sgu = ops.quantize_weights_fp8(inp.w_gate_up)
    qd, sd = ops.quantize_weights_fp8(inp.w_down)
    x, lg = cpu(inp.x), cpu(inp.logits)
    ref = oracle.moe_forward(x, lg, 2, cpu(inp.w_gate_up), cpu(inp.w_down), True)
    res = {}
    for mode in ("w8a16", "w8a8"):
        out = cpu(ops.fused_moe(inp.x, inp.logits, 2, qgu, qd, w_scales=(sgu, sd), out_dtype=torch.float32,
                                w8a8=(mode == "w8a8")))
        own = oracle.moe_forward_fp8(x, lg, 2, cpu(qgu), cpu(sgu), cpu(qd), cpu(sd), True, mode=mode)
        # the bf16 output, as the benchmark times it
        out16 = cpu(ops.fused_moe(inp.x, inp.logits, 2, qgu, qd, w_scales=(sgu, sd), w8a8=(mode == "w8a8"))).float()
        res[mode] = (oracle.rel_l2(out, ref), oracle.rel_l2(out, own), oracle.rel_l2(out16, ref))
        print("PARITY " + json.dumps({"case": f"mixtral-8x7b-fp8 {mode} T={T}", "rows": T,
                                      "rel_l2_vs_bf16_ref": res[mode][0], "rel_l2_vs_fp8_oracle": res[mode][1],
                                      "bf16_out_rel_l2_vs_bf16_ref": res[mode][2]},
                                     sort_keys=True), flush=True)
    assert res["w8a16"][1] <= 1e-2 and res["w8a8"][1] <= 1e-2
    assert res["w8a16"][0] <= 5e-2 and res["w8a16"][2] <= 5e-2
    assert res["w8a8"][0] <= 7.5e-2 and res["w8a8"][2] <= 7.5e-2


# The fp8 modes on cache-resident experts at a mid-size batch, at the real shapes (Qwen3-30B-A3B
# 32-expert share and DeepSeek-V2-Lite's routed experts, 768 tokens): the W8A16 LDS tiles that DMA
# the e4m3 weights and the tile rules for these launches, against the oracle's own fp8 forward.
@pytest.mark.parametrize("name", ["qwen3-30b-a3b-local32", "deepseek-v2-lite"])
def test_fp8_small_experts_real_shape(dev, name):
    import json
    T = 768
    s = SHAPES[name]
    inp = make_inputs(s, T, device=dev)
    qgu, sgu = ops.quantize_weights_fp8(inp.w_gate_up)
    qd, sd = ops.quantize_weights_fp8(inp.w_down)
    x, lg = cpu(inp.x), cpu(inp.logits)
    ref = oracle.moe_forward(x, lg, s.top_k, cpu(inp.w_gate_up), cpu(inp.w_down), s.renormalize,
                             expert_range=inp.expert_range)
    for mode in ("w8a16", "w8a8"):
        out = cpu(ops.fused_moe(inp.x, inp.logits, s.top_k, qgu, qd, renormalize=s.renormalize,
                                expert_range=inp.expert_range, w_scales=(sgu, sd), out_dtype=torch.float32,
                                w8a8=(mode == "w8a8")))
        own = oracle.moe_forward_fp8(x, lg, s.top_k, cpu(qgu), cpu(sgu), cpu(qd), cpu(sd), s.renormalize, mode=mode,
                                     expert_range=inp.expert_range)
        r_own, r_ref = oracle.rel_l2(out, own), oracle.rel_l2(out, ref)
        print("PARITY " + json.dumps({"case": f"{name} {mode} T={T} (routed experts)", "rows": T,
                                      "rel_l2_vs_bf16_ref": r_ref, "rel_l2_vs_fp8_oracle": r_own}, sort_keys=True),
              flush=True)
        assert r_own <= 1e-2
        assert r_ref <= (5e-2 if mode == "w8a16" else 7.5e-2)


# The W8A8 layer's activation quantisation does not depend on how the routing was obtained or on
# x's alignment (16-byte aligned rows take the register quantiser, others the two-pass one): the
# layer routed here, routed by the caller (EIMOE_ROUTING_IN) and run on x 8 bytes past a 16-byte
# boundary agree bit for bit; 1-256 tokens take the one-workgroup route+align, 300 and 1000 the
# other routing paths.
@pytest.mark.parametrize("T", [1, 5, 64, 256, 300, 1000])
def test_w8a8_layer_same_bytes_whatever_the_routing_path_and_x_alignment(dev, T):
    inp = make_inputs(SHAPES["mixtral-8x7b-fp8"], T, device="cpu", hidden=256, inter=256)
    qgu, sgu = oracle.quantize_weights_fp8(inp.w_gate_up.float())
    qd, sd = oracle.quantize_weights_fp8(inp.w_down.float())
    x, lg = inp.x.to(dev), inp.logits.to(dev)
    kw = dict(w_scales=(sgu.to(dev), sd.to(dev)), out_dtype=torch.float32, w8a8=True)
    out, ids, w = ops.fused_moe(x, lg, 2, qgu.to(dev), qd.to(dev), return_routing=True, **kw)
    routed_in = ops.fused_moe(x, None, 2, qgu.to(dev), qd.to(dev), routing=(ids, w), num_experts=8, **kw)
    assert torch.equal(cpu(out), cpu(routed_in))
    big = torch.empty(T * 256 + 4, dtype=torch.bfloat16, device=dev)
    x_odd = big[4:].view(T, 256)   # 8 bytes past a 16-byte boundary
    x_odd.copy_(x)
    assert x_odd.data_ptr() % 16 == 8
    odd = ops.fused_moe(x_odd, lg, 2, qgu.to(dev), qd.to(dev), **kw)
    assert torch.equal(cpu(out), cpu(odd))
    ref8 = oracle.moe_forward_fp8(inp.x, inp.logits, 2, qgu, sgu, qd, sd, True, mode="w8a8")
    assert oracle.rel_l2(cpu(out), ref8) <= 1e-2
