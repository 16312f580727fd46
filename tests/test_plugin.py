"""The drop-in expert module (HipFusedMoE), the MOE_IMPL registry and the torch.ops
op point.  Host logic runs on CPU; the forward tests are marked gpu."""
import numpy as np
import pytest
import torch

import oracle
from easyinfra_amd.moe import HipFusedMoE, SingleRankGroup, get_moe_impl


class _Group:
    def __init__(self, size, rank=0):
        self.group_size = size
        self.local_rank = rank


def test_get_moe_impl(monkeypatch):
    monkeypatch.setenv("MOE_IMPL", "hip")
    assert get_moe_impl() is HipFusedMoE
    monkeypatch.setenv("MOE_IMPL", "fused")
    assert get_moe_impl() is HipFusedMoE
    monkeypatch.setenv("MOE_IMPL", "cutlass")
    with pytest.raises(ValueError):
        get_moe_impl()
    monkeypatch.setenv("MOE_IMPL", "bogus")
    with pytest.raises(ValueError, match="Unrecognized"):
        get_moe_impl()


def test_constructor_checks_mirror_reference():
    phy = torch.arange(8).view(1, 8)
    m = HipFusedMoE(0, 64, 128, "silu", False, False, 8, SingleRankGroup(), SingleRankGroup(), phy)
    assert tuple(m.experts_gate_up_weight.shape) == (8, 256, 64)
    assert tuple(m.experts_down_weight.shape) == (8, 64, 128)
    assert m.forward == m.forward_noep
    with pytest.raises(ValueError, match="cannot divide"):
        HipFusedMoE(0, 64, 130, "silu", False, False, 8, SingleRankGroup(), _Group(4), phy)
    with pytest.raises(ValueError, match="devided"):
        HipFusedMoE(0, 64, 128, "silu", False, False, 9, _Group(2), SingleRankGroup(), torch.arange(4).view(2, 2))
    with pytest.raises(NotImplementedError):
        HipFusedMoE(0, 64, 128, "relu", False, False, 8, SingleRankGroup(), SingleRankGroup(), phy)
    with pytest.raises(NotImplementedError):
        HipFusedMoE(0, 64, 128, "silu", True, False, 8, SingleRankGroup(), SingleRankGroup(), phy)
    with pytest.raises(NotImplementedError):
        HipFusedMoE(0, 64, 128, "silu", False, True, 8, SingleRankGroup(), SingleRankGroup(), phy)
    # the reference's launcher takes `bias.stride(0) if bias else 0` (fused_moe.py:362): torch
    # refuses the truth value of a bias tensor, so its fused path raises with a bias as well
    bias = torch.zeros(8, 256)
    with pytest.raises(RuntimeError, match="ambiguous"):
        _ = bias.stride(0) if bias else 0
    ep = HipFusedMoE(0, 64, 128, "silu", False, False, 8, _Group(2, 1), SingleRankGroup(),
                     torch.arange(8).view(2, 4))
    assert ep.num_physical_experts == 4 and ep.forward == ep.forward_ep


def test_weight_loader_stacks_gate_up_like_reference():
    """fused_moe.py:91-101: [gate0, up0, gate1, up1, ...] -> [E, 2I, H]."""
    E, H, I = 3, 8, 4
    m = HipFusedMoE(0, H, I, "silu", False, False, E, phy2log_expert_map=torch.arange(E).view(1, E))
    g = torch.Generator().manual_seed(0)
    gates = [torch.randn(I, H, generator=g) for _ in range(E)]
    ups = [torch.randn(I, H, generator=g) for _ in range(E)]
    downs = [torch.randn(H, I, generator=g) for _ in range(E)]
    for e in reversed(range(E)):          # arrival order must not matter
        m.weight_loader("mlp.experts", ups[e], torch.float32, f"{e}.up_proj.weight")
        m.weight_loader("mlp.experts", downs[e], torch.float32, f"{e}.down_proj.weight")
        m.weight_loader("mlp.experts", gates[e], torch.float32, f"{e}.gate_proj.weight")
    assert not hasattr(m, "loaded_values")
    for e in range(E):
        assert torch.equal(m.experts_gate_up_weight[e, :I].cpu(), gates[e])
        assert torch.equal(m.experts_gate_up_weight[e, I:].cpu(), ups[e])
        assert torch.equal(m.experts_down_weight[e].cpu(), downs[e])
    with pytest.raises(ValueError):
        m.weight_loader("mlp.experts", gates[0], torch.float32, "0.gate_proj.weight")


def test_torch_op_schema_registered():
    import easyinfra_amd.torch_ops  # noqa: F401
    assert hasattr(torch.ops.ops, "hip_grouped_gemm_single")
    schema = str(torch.ops.ops.hip_grouped_gemm_single.default._schema)
    assert "Tensor[] B_list" in schema and "int[] block_sizes" in schema


# --------------------------------------------------------------------------- GPU
def _module(E, H, I, ep=1, dev="cuda"):
    g = torch.Generator().manual_seed(E * H)
    m = HipFusedMoE(0, H, I, "silu", False, False, E * ep, _Group(ep), SingleRankGroup(),
                    torch.arange(E * ep).view(ep, E))
    wgu = (torch.randn(E, 2 * I, H, generator=g) * 0.05).to(torch.bfloat16)
    wd = (torch.randn(E, H, I, generator=g) * 0.05).to(torch.bfloat16)
    m.experts_gate_up_weight = torch.nn.Parameter(wgu.to(dev), requires_grad=False)
    m.experts_down_weight = torch.nn.Parameter(wd.to(dev), requires_grad=False)
    return m, wgu, wd


@pytest.mark.gpu
@pytest.mark.parametrize("ep,as_list", [(1, False), (1, True), (2, True), (4, False)])
def test_forward_ep_matches_per_segment_oracle(dev, ep, as_list):
    E, H, I = 4, 128, 128
    m, wgu, wd = _module(E, H, I, ep, dev)
    g = torch.Generator().manual_seed(ep)
    counts = torch.randint(0, 40, (ep, E), generator=g)
    counts[0, 1] = 0
    M = int(counts.sum())
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    arg = counts.reshape(-1).tolist() if as_list else counts.to(dev)
    y = m.forward_ep(x.to(dev), arg).cpu().float()
    assert y.shape == (M, H)
    r = 0
    for s, c in enumerate(counts.reshape(-1).tolist()):
        e = s % E
        ref = oracle.expert_mlp(x[r:r + c].float(), wgu[e], wd[e], round_h_bf16=True)
        torch.testing.assert_close(y[r:r + c], ref, rtol=2e-2, atol=2e-2)
        r += c


@pytest.mark.gpu
def test_forward_ep_empty_input_returns_input(dev):
    m, _, _ = _module(4, 128, 128, 1, dev)
    x = torch.empty(0, 128, dtype=torch.bfloat16, device=dev)
    assert m.forward_ep(x, [0, 0, 0, 0]) is x


@pytest.mark.gpu
def test_forward_layer_and_fp8_weights(dev):
    E, H, I, T = 8, 128, 128, 64
    m, wgu, wd = _module(E, H, I, 1, dev)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    out = m.forward_layer(x.to(dev), logits.to(dev), 2, out_dtype=torch.float32).cpu()
    ref = oracle.moe_forward(x, logits, 2, wgu, wd, True)
    assert oracle.rel_l2(out, ref) <= 1e-2
    m.quantize_weights_fp8()
    out8 = m.forward_layer(x.to(dev), logits.to(dev), 2, out_dtype=torch.float32).cpu()
    qgu, sgu = oracle.quantize_weights_fp8(wgu.float())
    qd, sd = oracle.quantize_weights_fp8(wd.float())
    ref8 = oracle.moe_forward_fp8(x, logits, 2, qgu, sgu, qd, sd, True, mode="w8a16")
    assert oracle.rel_l2(out8, ref8) <= 1e-2
    assert oracle.rel_l2(out8, ref) <= 5e-2


@pytest.mark.gpu
def test_torch_op_matches_reference_contract(dev):
    import easyinfra_amd.torch_ops  # noqa: F401
    g = torch.Generator().manual_seed(8)
    K, N = 128, 192
    blocks = [5, 0, 70, 33]
    a = torch.randn(sum(blocks), K, generator=g).to(torch.bfloat16)
    bl = [(torch.randn(N, K, generator=g) * 0.1).to(torch.bfloat16) for _ in blocks]
    out = torch.ops.ops.hip_grouped_gemm_single(a.to(dev), [b.to(dev) for b in bl], blocks)
    ref = oracle.grouped_gemm(a, bl, blocks)
    assert out.dtype == torch.bfloat16
    torch.testing.assert_close(out.cpu().float(), ref, rtol=1e-2, atol=1e-2)


@pytest.mark.gpu
def test_torch_op_repeated_expert_list_reads_weights_in_place(dev):
    """The reference passes its experts' weights repeated ep_size times (single_group_gemm_moe.py:73-76):
    block i uses B_list[i]; the op must read the separate tensors where they lie (no stacked copy)."""
    import easyinfra_amd.torch_ops as tops
    g = torch.Generator().manual_seed(9)
    K, N, E, ep = 256, 128, 3, 2
    experts = [(torch.randn(N, K, generator=g) * 0.1).to(torch.bfloat16).to(dev) for _ in range(E)]
    bl = experts * ep
    blocks = [17, 0, 40, 3, 64, 9]
    a = torch.randn(sum(blocks), K, generator=g).to(torch.bfloat16)
    assert tops._period(bl) == E
    before = torch.cuda.memory_allocated(dev)
    out = torch.ops.ops.hip_grouped_gemm_single(a.to(dev), bl, blocks)
    grown = torch.cuda.memory_allocated(dev) - before
    assert grown < N * K * 2, f"op allocated {grown} bytes: looks like a weight copy"
    ref = oracle.grouped_gemm(a, [b.cpu() for b in bl], blocks)
    torch.testing.assert_close(out.cpu().float(), ref, rtol=1e-2, atol=1e-2)


def test_torch_op_period_detection():
    import easyinfra_amd.torch_ops as tops
    a, b, c = torch.zeros(2), torch.zeros(2), torch.zeros(2)
    assert tops._period([a, b, a, b]) == 2
    assert tops._period([a, b, c]) == 3
    assert tops._period([a, a, a]) == 1
    assert tops._period([a, b, a]) == 3
