"""Whole-layer parity: ops.fused_moe (one C-ABI call) against the CPU oracle.

Tolerances (bf16 path): rel-L2 <= 1e-2 against the fp32 oracle, max-abs <= 2e-2
on the fp32-output variant where the output magnitude allows it; and a tight
check against the oracle with h rounded to bf16 (the GPU path's storage
precision), which isolates accumulation-order noise.  Routing ids are bit-exact.

At the real (large) shapes the layer is evaluated for every token on the GPU and
compared row-by-row with the oracle on a seeded token subset (rows are
independent given the logits).
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


def _run(inp, dev, out_dtype=torch.float32, **kw):
    """The fused layer on the workload's own dtypes (fp32 workloads run the fp32 layer)."""
    s = inp.shape
    wgu, wd = inp.w_gate_up, inp.w_down
    sh_gu = inp.shared_gate_up.to(dev) if inp.shared_gate_up is not None else None
    sh_d = inp.shared_down.to(dev) if inp.shared_down is not None else None
    return ops.fused_moe(inp.x.to(dev), inp.logits.to(dev), s.top_k, wgu.to(dev), wd.to(dev),
                         renormalize=s.renormalize, shared_gate_up=sh_gu, shared_down=sh_d,
                         expert_range=inp.expert_range, out_dtype=out_dtype, return_routing=True, **kw)


def _oracle(inp, round_h=False, subset=None):
    s = inp.shape
    wgu, wd = inp.w_gate_up.cpu(), inp.w_down.cpu()
    sh_gu = inp.shared_gate_up.cpu() if inp.shared_gate_up is not None else None
    sh_d = inp.shared_down.cpu() if inp.shared_down is not None else None
    return oracle.moe_forward(inp.x.cpu(), inp.logits.cpu(), s.top_k, wgu, wd, s.renormalize, sh_gu, sh_d,
                              inp.expert_range, round_h_bf16=round_h, token_subset=subset)


@pytest.mark.parametrize("name", list(SHAPES))
@pytest.mark.parametrize("T", [1, 7, 96])
def test_layer_small_variant(dev, name, T):
    """Each workload's routing/expert structure at reduced H, I."""
    inp = make_inputs(SHAPES[name], T, device="cpu", hidden=256, inter=128)
    out, ids, w = _run(inp, dev)
    rid, rw = oracle.route_topk(inp.logits, inp.shape.top_k, inp.shape.renormalize)
    assert torch.equal(cpu(ids), rid)
    torch.testing.assert_close(cpu(w), rw, rtol=3e-6, atol=1e-7)
    got = cpu(out)
    ref = _oracle(inp)
    tight = _oracle(inp, round_h=True)
    assert oracle.rel_l2(got, ref) <= 1e-2
    assert float((got - ref).abs().max()) <= 2e-2
    if inp.x.dtype == torch.bfloat16:
        assert float((got - tight).abs().max()) <= 2e-3 * max(1.0, float(tight.abs().max()))
    else:   # the fp32 layer: fp32 operands on the fp32 MFMA, only the summation order differs
        assert oracle.rel_l2(got, ref) <= 2e-5
        assert float((got - ref).abs().max()) <= 1e-4 * max(1.0, float(ref.abs().max()))


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_layer_output_dtypes_and_y_fp32(dev, out_dtype):
    inp = make_inputs(SHAPES["deepseek-v2-lite"], 64, device="cpu", hidden=256, inter=128)
    a, _, _ = _run(inp, dev, out_dtype=out_dtype)
    b, _, _ = _run(inp, dev, out_dtype=out_dtype, y_fp32=True)
    ref = _oracle(inp)
    assert a.dtype == out_dtype
    assert oracle.rel_l2(cpu(a).float(), ref) <= 1e-2
    assert oracle.rel_l2(cpu(b).float(), ref) <= 1e-2


def test_layer_deterministic(dev):
    inp = make_inputs(SHAPES["qwen3-30b-a3b-local32"], 256, device="cpu", hidden=256, inter=128)
    a = _run(inp, dev)[0]
    b = _run(inp, dev)[0]
    assert torch.equal(a, b)


def test_layer_no_local_expert_rows_are_zero(dev):
    inp = make_inputs(SHAPES["qwen3-30b-a3b-local32"], 96, device="cpu", hidden=256, inter=128)
    out, ids, _ = _run(inp, dev)
    local = (cpu(ids) < 32).any(dim=1)
    assert (~local).any()
    assert torch.count_nonzero(cpu(out)[~local]) == 0


@pytest.mark.parametrize("T", [1, 77])
def test_layer_deepseek_v3_gate(dev, T):
    """The layer routed by the DeepSeek-V3 gate (sigmoid, correction bias, 8 groups keep 4,
    routed_scaling_factor) with shared experts, against the oracle on the same routing."""
    inp = make_inputs(SHAPES["deepseek-v2-lite"], T, device="cpu", hidden=256, inter=128)
    g = torch.Generator().manual_seed(T)
    bias = torch.randn(inp.logits.shape[1], generator=g) * 0.1
    kw = dict(scoring_func="sigmoid", n_group=8, topk_group=4, e_score_correction_bias=bias.to(dev),
              routed_scaling_factor=2.5)
    s = inp.shape
    out, ids, w = ops.fused_moe(inp.x.to(dev), inp.logits.to(dev), s.top_k, inp.w_gate_up.to(dev),
                                inp.w_down.to(dev), shared_gate_up=inp.shared_gate_up.to(dev),
                                shared_down=inp.shared_down.to(dev), out_dtype=torch.float32, return_routing=True, **kw)
    rid, rw = oracle.route_grouped_topk(inp.logits, s.top_k, 8, 4, bias, True, 2.5)
    assert torch.equal(cpu(ids), rid)
    torch.testing.assert_close(cpu(w), rw, rtol=2e-6, atol=1e-7)
    ref = oracle.moe_forward(inp.x.cpu(), inp.logits.cpu(), s.top_k, inp.w_gate_up.cpu(), inp.w_down.cpu(), True,
                             inp.shared_gate_up.cpu(), inp.shared_down.cpu(), routing=(rid, rw))
    assert oracle.rel_l2(cpu(out), ref) <= 1e-2
    # the same routing passed in explicitly (EIMOE_ROUTING_IN) gives the same output bit for bit
    out2 = ops.fused_moe(inp.x.to(dev), None, s.top_k, inp.w_gate_up.to(dev), inp.w_down.to(dev),
                         shared_gate_up=inp.shared_gate_up.to(dev), shared_down=inp.shared_down.to(dev),
                         out_dtype=torch.float32, routing=(ids, w), num_experts=inp.logits.shape[1])
    assert torch.equal(out, out2)


def test_layer_with_eplb_replicas_matches_logical_layer(dev):
    """Physical experts are copies of logical ones, so routing through the EPLB map (replica
    i mod count of each flat slot) onto physically laid-out weights reproduces the logical
    layer: router -> eplb_map -> fused layer with EIMOE_ROUTING_IN."""
    inp = make_inputs(SHAPES["qwen3-30b-a3b-local32"], 64, device="cpu", hidden=256, inter=128)
    s = inp.shape
    E = inp.logits.shape[1]
    wgu_log = torch.randn(E, 2 * 128, 256, generator=torch.Generator().manual_seed(1)) * 0.05
    wd_log = torch.randn(E, 256, 128, generator=torch.Generator().manual_seed(2)) * 0.05
    wgu_log, wd_log = wgu_log.to(torch.bfloat16).to(dev), wd_log.to(torch.bfloat16).to(dev)
    phy2log, log2phy, count = ops.eplb_default_layout(E, 4, E // 4 + 8)   # 8 replicas per rank
    flat = phy2log.reshape(-1).long().to(dev)
    x, lg = inp.x.to(dev), inp.logits.to(dev)
    ids, w = ops.router_topk(lg, s.top_k, s.renormalize)
    phys = ops.eplb_map(ids, log2phy.to(dev), count.to(dev))
    assert torch.equal(flat[phys.long()], ids.long())
    logical = ops.fused_moe(x, lg, s.top_k, wgu_log, wd_log, renormalize=s.renormalize, out_dtype=torch.float32)
    physical = ops.fused_moe(x, None, s.top_k, wgu_log[flat], wd_log[flat], out_dtype=torch.float32,
                             routing=(phys, w), num_experts=flat.numel())
    assert oracle.rel_l2(cpu(physical), cpu(logical)) <= 1e-5


# --------------------------------------------------------------------------- real shapes
REAL = [("tiny-mixtral-fp32", 512), ("mixtral-8x7b", 1), ("mixtral-8x7b", 8), ("mixtral-8x7b", 64),
        ("mixtral-8x7b", 8192), ("deepseek-v2-lite", 16), ("deepseek-v2-lite", 128), ("deepseek-v2-lite", 768),
        ("deepseek-v2-lite", 4096), ("qwen3-30b-a3b-local32", 1), ("qwen3-30b-a3b-local32", 32),
        ("qwen3-30b-a3b-local32", 256), ("qwen3-30b-a3b-local32", 768), ("qwen3-30b-a3b-local32", 1536),
        ("qwen3-30b-a3b-local32", 2048)]


def half_ulp_bf16(t: torch.Tensor) -> torch.Tensor:
    """Half a bf16 ulp at |t| (the most rounding a value to bf16 can move it)."""
    e = torch.floor(torch.log2(t.abs().clamp_min(2.0 ** -126)))
    return torch.pow(2.0, e - 8)


def parity_record(**kw):
    """One machine-readable line per real-shape check (collected into the committed parity table)."""
    import json
    print("PARITY " + json.dumps(kw, sort_keys=True), flush=True)


@pytest.mark.slow
@pytest.mark.parametrize("name,T", REAL)
def test_layer_real_shape(dev, name, T):
    """Every row of the layer at the workload's real shape against the fp32 oracle, in the default
    mode (the one the benchmark times: h = silu(g)*u stored in bf16, as the reference's intermediate
    cache; per-assignment outputs in fp32) and in the precise mode (h_split: h kept as two bf16 terms).

    Both modes: fp32 output within rel-L2 1e-2 and a fixed max-abs 2e-2 over all T*H values; bf16
    output within rel-L2 1e-2 and within 2e-2 + half a bf16 ulp elementwise (the fp32 result within
    2e-2, then one rounding to the output type)."""
    shape = SHAPES[name]
    inp = make_inputs(shape, T, device=dev)
    out, ids, w = _run(inp, dev)
    rid, rw = oracle.route_topk(cpu(inp.logits), shape.top_k, shape.renormalize)
    assert torch.equal(cpu(ids), rid)
    ref = _oracle(inp.to("cpu"))
    got = cpu(out)
    f32 = inp.x.dtype == torch.float32      # the fp32 layer: h is fp32 already, no precise mode
    precise = {} if f32 else {"h_split": True}
    got16 = cpu(_run(inp, dev, out_dtype=torch.bfloat16)[0]).float()
    gotp = cpu(_run(inp, dev, **precise)[0])
    gotp16 = cpu(_run(inp, dev, out_dtype=torch.bfloat16, **precise)[0]).float()

    def err(a):
        return oracle.rel_l2(a, ref), float((a - ref).abs().max())

    rel, mx = err(got)
    rel16, mx16 = err(got16)
    relp, mxp = err(gotp)
    relp16, mxp16 = err(gotp16)
    def excess(a):   # |a - ref| beyond the half ulp the rounding to bf16 may add
        return float(((a - ref).abs() - half_ulp_bf16(torch.maximum(ref.abs(), a.abs()))).max())

    excess16, excessp16 = excess(got16), excess(gotp16)
    parity_record(case=f"{name} T={T}", rows=T, values=got.numel(), max_ref=float(ref.abs().max()),
                  rel_l2=rel, max_abs=mx, bf16_rel_l2=rel16, bf16_max_abs=mx16, bf16_max_abs_minus_half_ulp=excess16,
                  precise_rel_l2=relp, precise_max_abs=mxp, precise_bf16_rel_l2=relp16, precise_bf16_max_abs=mxp16,
                  precise_bf16_max_abs_minus_half_ulp=excessp16)
    assert rel <= 1e-2 and mx <= 2e-2
    assert rel16 <= 1e-2 and excess16 <= 2e-2
    assert relp <= 1e-2 and mxp <= 2e-2
    assert relp16 <= 1e-2 and excessp16 <= 2e-2
    if f32:   # the reference's own precision: fp32 operands, only the summation order differs
        assert rel <= 2e-5 and mx <= 1e-4 * max(1.0, float(ref.abs().max()))


# The layer's own routing takes the router that writes the align's chunk counts (4-wave workgroups
# at 600 tokens, 8-wave ones at 1536 / 2040 / 2048 on a 32-of-128 expert window, the three-launch path
# at 2100); routing passed in takes the align alone.  Same output bit for bit, and the oracle's.
@pytest.mark.parametrize("T", [600, 1536, 2040, 2048, 2100])
def test_layer_routing_paths_agree(dev, T):
    inp = make_inputs(SHAPES["qwen3-30b-a3b-local32"], T, device="cpu", hidden=256, inter=256)
    s = inp.shape
    x, lg = inp.x.to(dev), inp.logits.to(dev)
    wgu, wd = inp.w_gate_up.to(dev), inp.w_down.to(dev)
    kw = dict(renormalize=s.renormalize, expert_range=inp.expert_range, out_dtype=torch.float32)
    out, ids, w = ops.fused_moe(x, lg, s.top_k, wgu, wd, return_routing=True, **kw)
    rid, _ = oracle.route_topk(inp.logits, s.top_k, s.renormalize)
    assert torch.equal(cpu(ids), rid)
    routed_in = ops.fused_moe(x, None, s.top_k, wgu, wd, routing=(ids, w), num_experts=s.n_experts, **kw)
    assert torch.equal(cpu(out), cpu(routed_in))
    assert oracle.rel_l2(cpu(out), _oracle(inp)) <= 1e-2


@pytest.mark.parametrize("name", ["mixtral-8x7b", "deepseek-v2-lite", "qwen3-30b-a3b-local32"])
@pytest.mark.parametrize("T", [1, 3, 200])
def test_layer_precise_mode_tracks_fp32(dev, name, T):
    """h_split keeps ~16 significant bits of h, so the layer tracks the fp32 oracle ~100x closer
    than the default bf16 intermediate (both routed and shared experts go through it)."""
    inp = make_inputs(SHAPES[name], T, device="cpu", hidden=256, inter=256)
    ref = _oracle(inp)
    scale = max(1.0, float(ref.abs().max()))
    p = cpu(_run(inp, dev, h_split=True)[0])
    d = cpu(_run(inp, dev)[0])
    assert oracle.rel_l2(p, ref) <= 5e-5
    assert float((p - ref).abs().max()) <= 2e-4 * scale
    assert oracle.rel_l2(p, ref) * 20 <= max(oracle.rel_l2(d, ref), 1e-6)


def test_block_prologue_then_v3_layer(dev):
    """The MoE block as a caller chains it: prologue (residual add, RMSNorm, fp32 router GEMM)
    then the layer with the DeepSeek-V3 gate and shared experts, against the oracle run on the
    GPU's own normed rows and logits (the prologue's parity is tested on its own)."""
    g = torch.Generator().manual_seed(11)
    T, H, I, E, k, Is = 100, 256, 128, 64, 6, 256
    hid = torch.randn(T, H, generator=g).to(torch.bfloat16)
    res = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ln = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    gate = (0.1 * torch.randn(E, H, generator=g)).to(torch.bfloat16)
    bias = 0.1 * torch.randn(E, generator=g)
    wgu = (0.05 * torch.randn(E, 2 * I, H, generator=g)).to(torch.bfloat16)
    wd = (0.05 * torch.randn(E, H, I, generator=g)).to(torch.bfloat16)
    sg = (0.05 * torch.randn(2 * Is, H, generator=g)).to(torch.bfloat16)
    sd = (0.05 * torch.randn(H, Is, generator=g)).to(torch.bfloat16)
    r = res.to(dev)
    r, normed, logits = ops.moe_prologue(hid.to(dev), r, ln.to(dev), 1e-6, gate.to(dev), logits_bf16=False,
                                         residual_out=r)
    out = ops.fused_moe(normed, logits, k, wgu.to(dev), wd.to(dev), scoring_func="sigmoid", n_group=8,
                        topk_group=4, e_score_correction_bias=bias.to(dev), routed_scaling_factor=2.5,
                        shared_gate_up=sg.to(dev), shared_down=sd.to(dev), out_dtype=torch.float32)
    ids, w = oracle.route_grouped_topk(cpu(logits), k, 8, 4, bias, True, 2.5)
    ref = oracle.moe_forward(cpu(normed), cpu(logits), k, wgu, wd, True, sg, sd, routing=(ids, w))
    assert oracle.rel_l2(cpu(out), ref) <= 1e-2


def test_fp32_hidden_states_on_bf16_weights_are_refused(dev):
    """fp32 activations run the fp32 layer with fp32 weights; on bf16 weights they are refused
    rather than rounded silently."""
    inp = make_inputs(SHAPES["mixtral-8x7b"], 4, device="cpu", hidden=256, inter=128)
    with pytest.raises(TypeError):
        ops.fused_moe(inp.x.float().to(dev), inp.logits.to(dev), 2, inp.w_gate_up.to(dev), inp.w_down.to(dev))


def test_fused_moe_refuses_mis_shaped_scales_and_shared_weights(dev):
    """Extents the kernels assume without reading them (per-channel scales, shared-expert weights,
    rows behind max_rows) are checked on the host: a wrong shape raises before any launch."""
    inp = make_inputs(SHAPES["mixtral-8x7b-fp8"], 8, device="cpu", hidden=256, inter=128)
    x, lg = inp.x.to(dev), inp.logits.to(dev)
    qgu, sgu = ops.quantize_weights_fp8(inp.w_gate_up.to(dev))
    qd, sd = ops.quantize_weights_fp8(inp.w_down.to(dev))
    for bad in [(sgu[:, :1].contiguous(), sd), (sgu, sd.reshape(-1)[:8].contiguous()), (sgu.reshape(-1), sd)]:
        with pytest.raises(ValueError):
            ops.fused_moe(x, lg, 2, qgu, qd, w_scales=bad)
    wgu, wd = inp.w_gate_up.to(dev), inp.w_down.to(dev)
    H, Is = 256, 128
    sg = torch.zeros(2 * Is, H, dtype=torch.bfloat16, device=dev)
    sdn = torch.zeros(H, Is, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.fused_moe(x, lg, 2, wgu, wd, shared_gate_up=sg[:Is].contiguous(), shared_down=sdn)
    with pytest.raises(ValueError):
        ops.fused_moe(x, lg, 2, wgu, wd, shared_gate_up=sg, shared_down=None)
    off = torch.tensor([0, 4, 8], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        ops.gemm_gate_up_silu(x[:4].contiguous(), wgu, off, 8)
    with pytest.raises(ValueError):
        ops.gemm_down(torch.zeros(4, 128, dtype=torch.bfloat16, device=dev), wd, off, 8)
    with pytest.raises(ValueError):
        ops.gemm_gate_up_silu(x, qgu, off, 8, w_scale=sgu[:1].contiguous())
    torch.cuda.synchronize()


@pytest.mark.parametrize("name,T", [("qwen3-30b-a3b-local32", 100), ("qwen3-30b-a3b-local32", 200),
                                    ("qwen3-30b-a3b-local32", 600), ("qwen3-30b-a3b-local32", 3000),
                                    ("deepseek-v2-lite", 600), ("deepseek-v2-lite", 700),
                                    ("deepseek-v2-lite", 4500), ("mixtral-8x7b", 500), ("mixtral-8x7b", 2900)])
def test_layer_routing_paths(dev, name, T):
    """Batch sizes that take each routing path of the fused layer: the one-workgroup router + align
    (up to 2 routing steps: Qwen3 100 tokens); the router writing each workgroup's per-expert counts
    then the many-workgroup align's placement, a chunk per router workgroup with a ragged last one
    (chunk-count matrices up to 2048 cells: Qwen3 200 and 600 tokens, Mixtral 500 and 2900); and with
    larger matrices the router then the one-workgroup align (below 4096 routed pairs: DeepSeek-V2-Lite
    600 tokens) or the two-pass many-workgroup align (Qwen3 3000, DeepSeek-V2-Lite 700 and 4500).
    Ids bit-exact, output against the oracle."""
    inp = make_inputs(SHAPES[name], T, device="cpu", hidden=128, inter=64)
    out, ids, w = _run(inp, dev)
    rid, rw = oracle.route_topk(inp.logits, inp.shape.top_k, inp.shape.renormalize)
    assert torch.equal(cpu(ids), rid)
    torch.testing.assert_close(cpu(w), rw, rtol=3e-6, atol=1e-7)
    ref = _oracle(inp, round_h=True)
    assert float((cpu(out) - ref).abs().max()) <= 2e-3 * max(1.0, float(ref.abs().max()))


# Full-size property: a token's output depends only on its own row and logits (routing per token,
# each GEMM row accumulated in the same K order whatever the other rows, the combine summing a
# token's slots in slot order), so permuting the tokens of a real-shape layer permutes its output
# bit for bit, in bf16 and in W8A8 (x quantised per token, h per routed row).  Per-expert row
# counts are unchanged by the permutation, so the same tiles run.
@pytest.mark.slow
@pytest.mark.parametrize("name,T,w8a8", [("mixtral-8x7b", 8192, False), ("mixtral-8x7b", 8192, True),
                                         ("deepseek-v2-lite", 4096, False), ("qwen3-30b-a3b-local32", 2048, False),
                                         ("mixtral-8x7b", 64, True), ("qwen3-30b-a3b-local32", 32, False)])
def test_layer_token_permutation_is_exact(dev, name, T, w8a8):
    shape = SHAPES[name]
    inp = make_inputs(shape, T, device=dev)
    kw = {}
    wgu, wd = inp.w_gate_up, inp.w_down
    if w8a8:
        wgu, sgu = ops.quantize_weights_fp8(wgu)
        wd, sd = ops.quantize_weights_fp8(wd)
        kw = dict(w_scales=(sgu, sd), w8a8=True)
    perm = torch.randperm(T, generator=torch.Generator().manual_seed(T)).to(dev)

    def run(x, lg):
        return ops.fused_moe(x, lg, shape.top_k, wgu, wd, renormalize=shape.renormalize,
                             shared_gate_up=inp.shared_gate_up, shared_down=inp.shared_down,
                             expert_range=inp.expert_range, out_dtype=torch.float32, **kw)

    base = run(inp.x, inp.logits)
    permuted = run(inp.x[perm].contiguous(), inp.logits[perm].contiguous())
    assert torch.equal(cpu(permuted), cpu(base)[cpu(perm)])


# Full-size sharding property: the layer over all experts equals the sum of the layers over disjoint
# expert windows (one GPU's share each, tokens without a resident expert giving zero rows), fp32
# outputs.  Not bit for bit: each window picks its own tiles and K split from its row counts, so the
# partial sums round differently; within rel-L2 1e-6.
@pytest.mark.slow
@pytest.mark.parametrize("name,T,windows", [("mixtral-8x7b", 8192, ((0, 2), (2, 4), (4, 6), (6, 8))),
                                            ("mixtral-8x7b", 64, ((0, 3), (3, 8))),
                                            ("deepseek-v2-lite", 4096, ((0, 16), (16, 48), (48, 64)))])
def test_layer_is_the_sum_of_its_expert_windows(dev, name, T, windows):
    shape = SHAPES[name]
    inp = make_inputs(shape, T, device=dev)
    E = shape.n_experts

    def run(lo, hi):
        return ops.fused_moe(inp.x, inp.logits, shape.top_k, inp.w_gate_up[lo:hi].contiguous(),
                             inp.w_down[lo:hi].contiguous(), renormalize=shape.renormalize,
                             expert_range=(lo, hi), out_dtype=torch.float32)

    full = cpu(run(0, E))
    parts = sum(cpu(run(lo, hi)) for lo, hi in windows)
    assert oracle.rel_l2(parts, full) <= 1e-6


# Every token routed to the same experts: a few long segments beside empty ones, on the prefill
# tiles (up to 256x256 with its persistent walk) and on the decode kernels.  Ids bit-exact, output
# against the oracle with h rounded to bf16 as the layer stores it.
@pytest.mark.parametrize("T,H,I,E,k,hot", [(3000, 256, 512, 8, 2, (5, 2)), (2048, 512, 256, 64, 6, (0, 1, 2, 3, 4, 5)),
                                           (40, 256, 256, 128, 8, (127, 3, 64, 9, 8, 100, 1, 77)),
                                           (1500, 128, 1024, 16, 1, (15,))])
def test_layer_all_tokens_on_the_same_experts(dev, T, H, I, E, k, hot):
    g = torch.Generator().manual_seed(T + E)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    for r, e in enumerate(hot):        # the same k experts on top of every row, in this order
        logits[:, e] = 20.0 - r
    w_gu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(torch.bfloat16)
    w_d = (torch.randn(E, H, I, generator=g) * 0.05).to(torch.bfloat16)
    out, ids, _ = ops.fused_moe(x.to(dev), logits.to(dev), k, w_gu.to(dev), w_d.to(dev), out_dtype=torch.float32,
                                return_routing=True)
    rid, _ = oracle.route_topk(logits, k, True)
    assert torch.equal(cpu(ids), rid)
    assert cpu(ids)[:, 0].eq(hot[0]).all()
    ref = oracle.moe_forward(x, logits, k, w_gu, w_d, True, round_h_bf16=True)
    assert float((cpu(out) - ref).abs().max()) <= 2e-3 * max(1.0, float(ref.abs().max()))


# Seeded random layer shapes: hidden and intermediate sizes, expert counts, top-k, token counts,
# expert-parallel windows, skewed routing and shared experts drawn so that the tile heuristic
# reaches the streaming kernel and every LDS tile (256x256 persistent, 128x128, 32x128, 16x64).
# Ids bit-exact with the oracle's router; the default mode within rel-L2 1e-2 of the fp32 oracle,
# the precise mode (h_split) within rel-L2 1e-2 and max-abs 2e-2; where H and I are multiples of
# 128 (and no shared experts), the W8A8 layer within rel-L2 1e-2 of the oracle's W8A8 forward.
@pytest.mark.parametrize("seed", list(range(80)))
def test_layer_random_shapes(dev, seed):
    rng = np.random.default_rng(1000 + seed)
    H = int(rng.choice([64, 128, 256, 512, 1024]))
    I = int(rng.choice([64, 128, 192, 256, 384, 512]))
    E = int(rng.choice([1, 2, 4, 8, 16, 40, 64, 96]))
    k = int(rng.integers(1, min(E, 8) + 1))
    T = int(rng.choice([1, 3, 17, 64, 100, 300, 700, 2000]))
    lo, hi = 0, E
    if E > 1 and rng.random() < 0.4:
        lo = int(rng.integers(0, E))
        hi = int(rng.integers(lo + 1, E + 1))
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    if rng.random() < 0.5:   # Zipf-like expert popularity
        logits += torch.log(1.0 / torch.arange(1, E + 1, dtype=torch.float32) ** 1.2)
    n_loc = hi - lo
    w_gu = (torch.randn(n_loc, 2 * I, H, generator=g) * 0.05).to(torch.bfloat16)
    w_d = (torch.randn(n_loc, H, I, generator=g) * 0.05).to(torch.bfloat16)
    sh_gu = sh_d = None
    if rng.random() < 0.25:
        Is = 64 * int(rng.integers(1, 5))
        sh_gu = (torch.randn(2 * Is, H, generator=g) * 0.05).to(torch.bfloat16)
        sh_d = (torch.randn(H, Is, generator=g) * 0.05).to(torch.bfloat16)
    er = (lo, hi) if (lo, hi) != (0, E) else None
    case = dict(seed=seed, T=T, H=H, I=I, E=E, k=k, window=(lo, hi), shared=sh_gu is not None)
    print("CASE", case, flush=True)

    def run(**kw):
        return ops.fused_moe(x.to(dev), logits.to(dev), k, w_gu.to(dev), w_d.to(dev),
                             shared_gate_up=None if sh_gu is None else sh_gu.to(dev),
                             shared_down=None if sh_d is None else sh_d.to(dev), expert_range=er,
                             out_dtype=torch.float32, return_routing=True, **kw)

    out, ids, _ = run()
    outp = run(h_split=True)[0]
    rid, _ = oracle.route_topk(logits, k, True)
    assert torch.equal(cpu(ids), rid), case
    ref = oracle.moe_forward(x, logits, k, w_gu, w_d, True, sh_gu, sh_d, er)
    assert oracle.rel_l2(cpu(out), ref) <= 1e-2, case
    gotp = cpu(outp)
    assert oracle.rel_l2(gotp, ref) <= 1e-2, case
    assert float((gotp - ref).abs().max()) <= 2e-2, case
    if H % 128 == 0 and I % 128 == 0 and sh_gu is None:
        qgu, sgu = oracle.quantize_weights_fp8(w_gu.float())
        qd, sd = oracle.quantize_weights_fp8(w_d.float())
        out8 = ops.fused_moe(x.to(dev), logits.to(dev), k, qgu.to(dev), qd.to(dev), expert_range=er,
                             w_scales=(sgu.to(dev), sd.to(dev)), out_dtype=torch.float32, w8a8=True)
        ref8 = oracle.moe_forward_fp8(x, logits, k, qgu, sgu, qd, sd, True, mode="w8a8", expert_range=er)
        assert oracle.rel_l2(cpu(out8), ref8) <= 1e-2, case


def test_release_streams_then_layer_again(dev):
    """The shared experts' second stream released between two calls: the second call creates it
    again and gives the same output bit for bit; the current device is kept."""
    inp = make_inputs(SHAPES["deepseek-v2-lite"], 300, device="cpu", hidden=256, inter=128)
    a = _run(inp, dev)[0]
    torch.cuda.synchronize()
    before = torch.cuda.current_device()
    ops.release_streams()
    assert torch.cuda.current_device() == before
    ops.release_streams()   # nothing left to release: still fine
    b = _run(inp, dev)[0]
    assert torch.equal(a, b)
