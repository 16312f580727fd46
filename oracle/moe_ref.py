"""CPU oracle for the fused-MoE expert path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
reference results are compared with (or, in the bench, as the timed CPU
baseline).  The product path
(``easyinfra_amd``) never calls it; it fails loudly when its HIP library is
missing.

This is a restatement of EasyInfra's single-GPU (ep=1) MoE layer semantics,
with every collective replaced by the identity it is at group size 1
(easyinfra/generation/parallel/communicator.py:143-148, 168-172, 270-271):

  route_topk     modeling_qwen3_moe.py:255-266 (softmax -> top-k -> renorm)
  route_grouped_topk  modeling_deepseek_v3.py:151-203 (DeepSeek-V3 gate: sigmoid,
                 correction bias, group-limited top-k, renorm, scaling)
  eplb_map       blocks/moe/base.py:40-64 (EPLB logical -> physical replica ids)
  moe_prologue   moe_all2all.py:329-336 (residual add), base_rmsnorm.py:6-12 (RMSNorm),
                 base_linear.py:28-36 / modeling_deepseek_v3.py:155-157 (router logits)
  align          blocks/moe/base.py:343-364 (per-expert counts),
                 moe_all2all.py:346-348 (sort, token index, slot), with the
                 EP-local expert window of blocks/moe/base.py:162-169, 187
  gather         moe_all2all.py:351
  expert_mlp     modules/moe/base.py:39-42, native_moe.py:56-103,
                 fused_moe.py:445-476 (gate/up -> silu(g)*u -> down)
  combine        moe_all2all.py:291-307 (weighted index_add_)
  shared_mlp     blocks/mlp.py:78-81 (+ modeling_deepseek_v3.py:213 sizing)
  moe_forward    moe_all2all.py:85-95 stages composed (a14)

Two deliberate, documented choices where the reference is not reproducible:
  * Top-k ties: the reference's ``torch.topk`` tie order is implementation
    defined.  The oracle selects by logit value (softmax is monotonic), ties to
    the lower expert id.
  * Sort stability: ``torch.sort(stable=False)`` (moe_all2all.py:346) promises
    no order among equal experts.  The oracle pins the stable order
    (expert, then flat index t*k+slot).

fp8 helpers (weight per-output-channel absmax/448 scales, per-token dynamic
activation scales, OCP e4m3fn with round-to-nearest-even as torch's CPU cast)
have no counterpart in the reference (fused_moe.py:331-335 maps fp8 inputs to
a bf16 compute type and takes no scales).

Pinning: every function here is checked in tests/test_oracle.py against an
independent formulation (brute-force loops on tiny shapes, a dense
all-experts-masked formulation, float64 closed forms, invariants), not by
re-typing the formula.
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

FP8_MAX = 448.0


# --------------------------------------------------------------------------- router
def route_topk(logits: torch.Tensor, k: int, renormalize: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """modeling_qwen3_moe.py:255-266.

    probs = softmax(logits, fp32); ids = top-k (canonical: by logit, ties -> lower id);
    w = probs[ids], renormalised over the k picks when ``renormalize``.
    Returns (ids int32 [T,k], w fp32 [T,k]).  Weights stay fp32 (the reference casts
    them to the activation dtype before the combine; the oracle keeps fp32).
    """
    logits = torch.as_tensor(logits).to(torch.float32)
    probs = torch.softmax(logits, dim=-1, dtype=torch.float32)
    ids = torch.sort(-logits, dim=-1, stable=True).indices[:, :k]
    w = probs.gather(1, ids)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return ids.to(torch.int32), w


def sigmoid_rn(logits) -> np.ndarray:
    """fp32 sigmoid rounded once from float64: the correctly rounded value (barring a float64
    result within its own error of an fp32 rounding boundary)."""
    x = np.asarray(logits, dtype=np.float64)
    with np.errstate(over="ignore"):
        return (1.0 / (1.0 + np.exp(-x))).astype(np.float32)


def route_grouped_topk(logits, k: int, n_group: int, topk_group: int, bias=None, renormalize: bool = True,
                       scaling: float = 1.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """DeepseekV3MoEGate.forward with topk_method "noaux_tc" and scoring "sigmoid"
    (modeling_deepseek_v3.py:151-203), from the fp32 logits on:

      scores = sigmoid(logits)                                   (:157-158)
      c = scores + e_score_correction_bias                       (:167)
      group score = sum of the top 2 of c in each group          (:168-170)
      keep topk_group groups; c := 0 outside them (masked_fill)  (:171-186)
      ids = top-k of c; w = scores[ids]                          (:187-190)
      w /= w.sum() + 1e-20 when norm_topk_prob and k > 1          (:196-198)
      w *= routed_scaling_factor                                 (:199)

    Deliberate choices where the reference is not reproducible: the sigmoid is the
    correctly rounded fp32 value (``sigmoid_rn``; the reference's fp32 ``torch.sigmoid``
    can differ by an ulp, which changes a pick only at an exact near-tie); both top-k
    steps use ``sorted=False`` in the reference, so their tie order is implementation
    defined: here groups and experts tie to the lower index, and the picks are listed
    in descending order of c.  Weights stay fp32 (the reference casts them to the
    activation dtype).  Returns (ids int32 [T,k], w fp32 [T,k]).
    """
    lg = np.asarray(torch.as_tensor(logits).float())
    T, E = lg.shape
    gsize = E // n_group
    s = sigmoid_rn(lg)
    b = np.zeros(E, np.float32) if bias is None else np.asarray(torch.as_tensor(bias).float())
    c = (s + b[None, :]).astype(np.float32)
    grp = np.sort(c.reshape(T, n_group, gsize), axis=-1)
    gscore = (grp[..., -1] + grp[..., -2]).astype(np.float32)          # top-1 + top-2, fp32
    keys = np.arange(n_group)
    ids = np.zeros((T, k), np.int64)
    w = np.zeros((T, k), np.float32)
    for t in range(T):
        gorder = sorted(keys, key=lambda g: (-float(gscore[t, g]), g))
        keep = np.zeros(n_group, bool)
        keep[gorder[:topk_group]] = True
        cm = np.where(np.repeat(keep, gsize), c[t], np.float32(0.0))
        order = sorted(range(E), key=lambda e: (-float(cm[e]), e))[:k]
        ids[t] = order
        w[t] = s[t, order]
    if renormalize and k > 1:
        w = (w / (w.sum(axis=-1, keepdims=True, dtype=np.float32) + np.float32(1e-20))).astype(np.float32)
    w = (w * np.float32(scaling)).astype(np.float32)
    return torch.from_numpy(ids.astype(np.int32)), torch.from_numpy(w)


def eplb_map(ids, log2phy, replica_count) -> torch.Tensor:
    """eplb_map_to_physical_and_record (generation/blocks/moe/base.py:40-64): flat slot i of
    the [T,k] ids takes replica i % replica_count[id] of its logical expert.  Ids outside
    [0, L) map to -1 (the reference would index out of range)."""
    ids = np.asarray(torch.as_tensor(ids)).astype(np.int64)
    l2p = np.asarray(torch.as_tensor(log2phy)).astype(np.int64)
    cnt = np.asarray(torch.as_tensor(replica_count)).astype(np.int64)
    flat = ids.reshape(-1)
    out = np.full(flat.shape, -1, np.int64)
    for i, l in enumerate(flat):
        if 0 <= l < l2p.shape[0] and 1 <= cnt[l] <= l2p.shape[1]:
            out[i] = l2p[l, i % cnt[l]]
    return torch.from_numpy(out.reshape(ids.shape).astype(np.int32))


def moe_prologue(hidden, residual, norm_w, eps: float, gate_w, logits_bf16: bool = True):
    """The MoE block's prologue: MoeAll2AllBlock.all2all_chunk_routing_compute
    (generation/blocks/moe/moe_all2all.py:329-336):
      residual = residual + hidden                           (compute_utils.py:14, bf16)
      normed = _rmsnorm(residual, weight, eps)               (base_rmsnorm.py:6-12):
               t = r.float(); t = t * rsqrt(mean(t^2) + eps); weight * t.to(bf16)
      logits = F.linear(normed, gate_w)                      (base_linear.py:28-36, bf16: Qwen3,
               Mixtral)  or  F.linear(normed.float(), gate_w.float())  (DeepseekV3MoEGate,
               modeling_deepseek_v3.py:155-157)
    bf16 tensors in, (residual [T,H] bf16, normed [T,H] bf16, logits [T,E] fp32) out."""
    hidden = torch.as_tensor(hidden).to(torch.bfloat16)
    residual = torch.as_tensor(residual).to(torch.bfloat16)
    norm_w = torch.as_tensor(norm_w).to(torch.bfloat16)
    gate_w = torch.as_tensor(gate_w).to(torch.bfloat16)
    r = residual + hidden
    t = r.to(torch.float32)
    variance = t.pow(2).mean(-1, keepdim=True)
    t = t * torch.rsqrt(variance + eps)
    normed = norm_w * t.to(torch.bfloat16)
    if logits_bf16:
        logits = F.linear(normed, gate_w).float()
    else:
        logits = F.linear(normed.float(), gate_w.float())
    return r, normed, logits


# --------------------------------------------------------------------------- align
def align(ids: np.ndarray, n_local: int, e_lo: int = 0):
    """Counts, offsets, stable expert-major permutation and its inverse.

    blocks/moe/base.py:343-364: counts = zeros(E).scatter_add_(ids, 1), restricted to
    the local window [e_lo, e_lo+n_local) (base.py:187).  moe_all2all.py:346-348:
    sorted flat positions, token = flat // k, slot = flat % k.

    Returns dict of int32 numpy arrays: counts[n_local], offsets[n_local+1],
    sorted_flat[A], sorted_tok[A], pos[T*k] (row of each flat slot, -1 if not local).
    """
    ids = np.asarray(ids)
    T, k = ids.shape
    flat = ids.reshape(-1).astype(np.int64) - e_lo
    local = (flat >= 0) & (flat < n_local)
    counts = np.bincount(flat[local], minlength=n_local).astype(np.int64)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    idx = np.nonzero(local)[0]
    order = idx[np.argsort(flat[idx], kind="stable")]
    pos = np.full(T * k, -1, dtype=np.int64)
    pos[order] = np.arange(order.size)
    return {
        "counts": counts.astype(np.int32),
        "offsets": offsets.astype(np.int32),
        "sorted_flat": order.astype(np.int32),
        "sorted_tok": (order // k).astype(np.int32),
        "sorted_slot": (order % k).astype(np.int32),
        "pos": pos.astype(np.int32),
    }


def gather(x: torch.Tensor, sorted_tok) -> torch.Tensor:
    """moe_all2all.py:351: send_hidden_states = h[send_indices]."""
    return x[torch.as_tensor(np.asarray(sorted_tok), dtype=torch.long)]


# --------------------------------------------------------------------------- experts
def silu(x: torch.Tensor) -> torch.Tensor:
    """activation/base_activation.py:8-11 (torch.nn.SiLU): x * sigmoid(x)."""
    return x * torch.sigmoid(x)


def _round_bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float32)


def expert_mlp(xs: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor,
               round_h_bf16: bool = False) -> torch.Tensor:
    """One expert: modules/moe/base.py:39-42 / fused_moe.py:445-476, fp32 math.

    gu = xs @ W_gu^T (rows [0,I) gate, [I,2I) up); h = silu(g) * u; y = h @ W_d^T.
    ``round_h_bf16`` rounds h to bf16 before the down projection, the storage
    precision of the GPU path's intermediate (used for tighter checks only).
    """
    I = w_down.shape[1]
    gu = F.linear(xs.float(), w_gate_up.float())
    h = silu(gu[:, :I]) * gu[:, I:]
    if round_h_bf16:
        h = _round_bf16(h)
    return F.linear(h, w_down.float())


def shared_mlp(x: torch.Tensor, shared_gate_up: torch.Tensor, shared_down: torch.Tensor,
               round_h_bf16: bool = False) -> torch.Tensor:
    """blocks/mlp.py:78-81: a dense SwiGLU MLP, weight 1.0, added to the layer output."""
    return expert_mlp(x, shared_gate_up, shared_down, round_h_bf16)


def moe_forward(x: torch.Tensor, logits: torch.Tensor, k: int, w_gate_up: torch.Tensor,
                w_down: torch.Tensor, renormalize: bool = True,
                shared_gate_up: Optional[torch.Tensor] = None, shared_down: Optional[torch.Tensor] = None,
                expert_range: Optional[Tuple[int, int]] = None, round_h_bf16: bool = False,
                token_subset: Optional[torch.Tensor] = None, return_parts: bool = False,
                routing: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
    """The layer at ep=1 (moe_all2all.py:85-95): route -> align -> gather -> experts -> combine.

    ``expert_range=(lo,hi)`` keeps only assignments to experts [lo,hi) (one GPU's EP
    share, blocks/moe/base.py:162-169); ``w_gate_up/w_down`` then hold those experts
    only.  Tokens with no local expert produce zero rows.  ``token_subset`` evaluates
    only the given token rows (the layer is row-independent given the logits).
    ``routing=(ids, w)`` replaces the softmax router (e.g. with ``route_grouped_topk``).
    Returns fp32 [T or |subset|, H].
    """
    x = torch.as_tensor(x)
    logits = torch.as_tensor(logits).float()
    if token_subset is not None:
        token_subset = torch.as_tensor(token_subset, dtype=torch.long)
        x, logits = x[token_subset], logits[token_subset]
        if routing is not None:
            routing = (routing[0][token_subset], routing[1][token_subset])
    T, H = x.shape
    ids, w = routing if routing is not None else route_topk(logits, k, renormalize)
    lo, hi = expert_range if expert_range is not None else (0, w_gate_up.shape[0])
    al = align(ids.numpy(), hi - lo, lo)
    out = torch.zeros(T, H, dtype=torch.float32)
    xs = gather(x, al["sorted_tok"]).float()
    tok = torch.as_tensor(al["sorted_tok"], dtype=torch.long)
    slot = torch.as_tensor(al["sorted_slot"], dtype=torch.long)
    w_sorted = w[tok, slot]                                   # moe_all2all.py:193
    ys = torch.empty(xs.shape[0], H, dtype=torch.float32)
    off = al["offsets"]
    for e in range(hi - lo):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            ys[a:b] = expert_mlp(xs[a:b], w_gate_up[e], w_down[e], round_h_bf16)
    out.index_add_(0, tok, ys * w_sorted[:, None])            # moe_all2all.py:302-304
    if shared_gate_up is not None:
        out += shared_mlp(x.float(), shared_gate_up, shared_down, round_h_bf16)
    if return_parts:
        return out, {"ids": ids, "w": w, "align": al, "ys": ys}
    return out


def moe_forward_dense(x, logits, k, w_gate_up, w_down, renormalize=True, shared_gate_up=None,
                      shared_down=None, expert_range=None) -> torch.Tensor:
    """Independent formulation used only to pin ``moe_forward``: every token through
    every local expert, combined with a dense [T,E] gate matrix (zeros off the top-k),
    float64 throughout.  No sort, no gather, no index_add_."""
    x = torch.as_tensor(x).double()
    logits = torch.as_tensor(logits).double()
    T, E = logits.shape
    lo, hi = expert_range if expert_range is not None else (0, w_gate_up.shape[0])
    p = torch.softmax(logits, dim=-1)
    gate = torch.zeros(T, E, dtype=torch.float64)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-float(logits[t, e]), e))[:k]
        sel = torch.tensor(order)
        wt = p[t, sel]
        if renormalize:
            wt = wt / wt.sum()
        gate[t, sel] = wt
    I = w_down.shape[2]
    out = torch.zeros(T, x.shape[1], dtype=torch.float64)
    for e in range(hi - lo):
        gu = x @ w_gate_up[e].double().T
        h = gu[:, :I] * torch.sigmoid(gu[:, :I]) * gu[:, I:]
        out += gate[:, lo + e:lo + e + 1] * (h @ w_down[e].double().T)
    if shared_gate_up is not None:
        Is = shared_down.shape[1]
        gu = x @ shared_gate_up.double().T
        out += (gu[:, :Is] * torch.sigmoid(gu[:, :Is]) * gu[:, Is:]) @ shared_down.double().T
    return out


# --------------------------------------------------------------------------- fp8
def quantize_rows_fp8(t: torch.Tensor):
    """Per-row absmax/448 scale and OCP e4m3fn values (torch CPU cast, RNE).

    Used for weights (one scale per output channel = per row of [E*N, K]) and for
    activations (one scale per token).  Returns (q float8_e4m3fn, scale fp32 [rows]).
    A zero row gets scale 1 (its values quantise to 0 either way).
    """
    t32 = t.float()
    amax = t32.abs().amax(dim=-1)
    scale = amax / FP8_MAX
    scale = torch.where(amax > 0, scale, torch.ones_like(scale))
    q = (t32 / scale.unsqueeze(-1)).to(torch.float8_e4m3fn)
    return q, scale


def quantize_weights_fp8(w: torch.Tensor):
    """[E,N,K] -> (q [E,N,K] e4m3fn, scale [E,N] fp32): per-output-channel scales."""
    E, N, K = w.shape
    q, s = quantize_rows_fp8(w.reshape(E * N, K))
    return q.view(E, N, K), s.view(E, N)


def gate_up_fp8(xs, wq_gu, s_gu, mode: str = "w8a8") -> torch.Tensor:
    """The fp8 gate/up projection of one expert, fp32 [rows, 2I] (before SiLU*mul).

    w8a16: gu = (x @ Wq^T) * s_gu[None, :], x in bf16-exact fp32.
    w8a8:  x quantised per token first: gu = (xq @ Wq^T) * s_x[:, None] * s_gu[None, :].
    """
    wgu = wq_gu.float()
    if mode == "w8a8":
        xq, sx = quantize_rows_fp8(xs)
        return (xq.float() @ wgu.T) * sx[:, None] * s_gu[None, :]
    return (xs.float() @ wgu.T) * s_gu[None, :]


def expert_mlp_fp8(xs, wq_gu, s_gu, wq_d, s_d, mode: str = "w8a8") -> torch.Tensor:
    """One expert with fp8 weights.

    w8a16: y = (silu(g)*u rounded to bf16) @ Wq_d^T * s_d, gate/up as in ``gate_up_fp8``.
    w8a8:  h = silu(g)*u is stored in bf16 (the expert path's intermediate precision) and
           quantised per row from that copy: y = (hq @ Wq_d^T) * s_h[:, None] * s_d[None, :].
    """
    I = wq_d.shape[1]
    wd = wq_d.float()
    gu = gate_up_fp8(xs, wq_gu, s_gu, mode)
    h = _round_bf16(silu(gu[:, :I]) * gu[:, I:])
    if mode == "w8a8":
        hq, sh = quantize_rows_fp8(h)
        return (hq.float() @ wd.T) * sh[:, None] * s_d[None, :]
    return (h @ wd.T) * s_d[None, :]


def moe_forward_fp8(x, logits, k, wq_gu, s_gu, wq_d, s_d, renormalize=True, mode="w8a8",
                    expert_range=None, token_subset=None) -> torch.Tensor:
    """moe_forward with fp8 expert weights (see expert_mlp_fp8)."""
    x = torch.as_tensor(x)
    logits = torch.as_tensor(logits).float()
    if token_subset is not None:
        token_subset = torch.as_tensor(token_subset, dtype=torch.long)
        x, logits = x[token_subset], logits[token_subset]
    T, H = x.shape
    ids, w = route_topk(logits, k, renormalize)
    lo, hi = expert_range if expert_range is not None else (0, wq_gu.shape[0])
    al = align(ids.numpy(), hi - lo, lo)
    tok = torch.as_tensor(al["sorted_tok"], dtype=torch.long)
    slot = torch.as_tensor(al["sorted_slot"], dtype=torch.long)
    xs = x[tok].float()
    ys = torch.empty(xs.shape[0], H, dtype=torch.float32)
    off = al["offsets"]
    for e in range(hi - lo):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            ys[a:b] = expert_mlp_fp8(xs[a:b], wq_gu[e], s_gu[e], wq_d[e], s_d[e], mode)
    out = torch.zeros(T, H, dtype=torch.float32)
    out.index_add_(0, tok, ys * w[tok, slot][:, None])
    return out


# --------------------------------------------------------------------------- grouped GEMM
def grouped_gemm(a: torch.Tensor, b_list, block_sizes) -> torch.Tensor:
    """single_group_gemm_moe.py:76-91 contract: out[rows_i] = A[rows_i] @ B_i^T over
    contiguous row blocks, B_i in nn.Linear layout [N,K]; fp32 result."""
    outs, r = [], 0
    for b, n in zip(b_list, block_sizes):
        outs.append(F.linear(a[r:r + n].float(), b.float()))
        r += n
    return torch.cat(outs, 0) if outs else a.new_zeros(0, b_list[0].shape[0], dtype=torch.float32)


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double()
    b = b.double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))
