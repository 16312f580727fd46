"""Committed fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the pinned oracle): the oracle must keep reproducing them (CPU), and the
HIP path must match them (GPU): routing and permutation bit-exact, the layer
output within the bf16 tolerance."""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

GOLD = Path(__file__).resolve().parent / "golden"
ROUTING = sorted(GOLD.glob("routing_*.npz"))
LAYERS = sorted(GOLD.glob("layer_*.npz"))


def _bf16(a):
    return torch.from_numpy(a).view(torch.bfloat16)


@pytest.mark.parametrize("path", ROUTING, ids=lambda p: p.stem)
def test_oracle_reproduces_routing_fixture(path):
    f = np.load(path)
    ids, w = oracle.route_topk(torch.from_numpy(f["logits"]), int(f["top_k"]), bool(f["renormalize"]))
    assert np.array_equal(ids.numpy(), f["ids"])
    np.testing.assert_allclose(w.numpy(), f["weights"], rtol=1e-6, atol=1e-9)
    al = oracle.align(ids.numpy(), int(f["n_local"]), int(f["e_lo"]))
    for k in ("counts", "offsets", "sorted_flat", "sorted_tok", "pos"):
        assert np.array_equal(al[k], f[k]), k


@pytest.mark.parametrize("path", LAYERS, ids=lambda p: p.stem)
def test_oracle_reproduces_layer_fixture(path):
    f = np.load(path)
    out = oracle.moe_forward(_bf16(f["x_bf16"]), torch.from_numpy(f["logits"]), int(f["top_k"]),
                             _bf16(f["w_gate_up_bf16"]), _bf16(f["w_down_bf16"]), bool(f["renormalize"]))
    np.testing.assert_allclose(out.numpy(), f["out"], rtol=1e-5, atol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("path", ROUTING, ids=lambda p: p.stem)
def test_gpu_routing_matches_fixture(dev, path):
    from easyinfra_amd import ops
    f = np.load(path)
    ids, w = ops.router_topk(torch.from_numpy(f["logits"]).to(dev), int(f["top_k"]), bool(f["renormalize"]))
    assert np.array_equal(ids.cpu().numpy(), f["ids"])
    np.testing.assert_allclose(w.cpu().numpy(), f["weights"], rtol=3e-6, atol=1e-7)
    al = ops.align(ids, int(f["n_local"]), int(f["e_lo"]))
    A = int(f["offsets"][-1])
    assert np.array_equal(al["counts"].cpu().numpy(), f["counts"])
    assert np.array_equal(al["offsets"].cpu().numpy(), f["offsets"])
    assert np.array_equal(al["sorted_flat"].cpu().numpy()[:A], f["sorted_flat"])
    assert np.array_equal(al["sorted_tok"].cpu().numpy()[:A], f["sorted_tok"])
    assert np.array_equal(al["pos"].cpu().numpy(), f["pos"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", LAYERS, ids=lambda p: p.stem)
def test_gpu_layer_matches_fixture(dev, path):
    from easyinfra_amd import ops
    f = np.load(path)
    out = ops.fused_moe(_bf16(f["x_bf16"]).to(dev), torch.from_numpy(f["logits"]).to(dev), int(f["top_k"]),
                        _bf16(f["w_gate_up_bf16"]).to(dev), _bf16(f["w_down_bf16"]).to(dev),
                        renormalize=bool(f["renormalize"]), out_dtype=torch.float32)
    ref = torch.from_numpy(f["out"])
    got = out.cpu()
    assert oracle.rel_l2(got, ref) <= 1e-2
    assert float((got - ref).abs().max()) <= 2e-2
