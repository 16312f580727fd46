"""Writes the committed fixtures in this directory from the CPU oracle.

The reference has no golden vectors for this path; these fixtures freeze the
pinned oracle's outputs (tests/test_oracle.py) on small seeded inputs so the GPU
path and any later change to the oracle are checked against fixed data.

  routing_*.npz  logits -> top-k ids/weights, counts, offsets, stable permutation
                 (DeepSeek-V2-Lite 64-expert Zipf router, Qwen3 128-expert router
                 with a 32-expert local window, Mixtral 8-expert router)
  layer_*.npz    full layer (bf16 inputs, fp32 output) for 8-expert layers

Run from the repository root:  python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from easyinfra_amd.workloads import SHAPES, make_inputs  # noqa: E402

OUT = Path(__file__).resolve().parent


def bf16_bits(t):
    return t.to(torch.bfloat16).view(torch.int16).numpy()


def routing_fixture(name, T, fname):
    s = SHAPES[name]
    inp = make_inputs(s, T, device="cpu", hidden=64, inter=64)
    ids, w = oracle.route_topk(inp.logits, s.top_k, s.renormalize)
    lo, hi = (0, s.e_loc)
    al = oracle.align(ids.numpy(), hi - lo, lo)
    np.savez_compressed(OUT / fname, logits=inp.logits.numpy(), top_k=s.top_k, renormalize=s.renormalize,
                        e_lo=lo, n_local=hi - lo, ids=ids.numpy(), weights=w.numpy(), **{
                            k: v for k, v in al.items()})


def layer_fixture(name, T, fname):
    s = SHAPES[name]
    inp = make_inputs(s, T, device="cpu", hidden=128, inter=64)
    x = inp.x.to(torch.bfloat16)
    wgu = inp.w_gate_up.to(torch.bfloat16)
    wd = inp.w_down.to(torch.bfloat16)
    out = oracle.moe_forward(x, inp.logits, s.top_k, wgu, wd, s.renormalize)
    np.savez_compressed(OUT / fname, x_bf16=bf16_bits(x), logits=inp.logits.numpy(), w_gate_up_bf16=bf16_bits(wgu),
                        w_down_bf16=bf16_bits(wd), top_k=s.top_k, renormalize=s.renormalize, out=out.numpy())


def main():
    torch.manual_seed(0)
    routing_fixture("deepseek-v2-lite", 64, "routing_deepseek_v2_lite.npz")
    routing_fixture("qwen3-30b-a3b-local32", 64, "routing_qwen3_local32.npz")
    routing_fixture("mixtral-8x7b", 96, "routing_mixtral.npz")
    layer_fixture("mixtral-8x7b", 48, "layer_mixtral_small.npz")
    layer_fixture("tiny-mixtral-fp32", 32, "layer_tiny_mixtral.npz")
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)


if __name__ == "__main__":
    main()
