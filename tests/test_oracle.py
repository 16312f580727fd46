"""Pins the CPU oracle (CPU-only tests).

The reference ships no tests, golden vectors or fixtures for this path, so each
oracle function is checked against an independent statement of the same math:
brute-force loops in float64, the reference's literal torch ops where they are
deterministic, closed forms, and invariants (EP decomposition, linearity,
permutation identities) chosen so that a dropped term, a wrong index or a
swapped operand fails at least one check.
"""
import math

import numpy as np
import pytest
import torch

import oracle
from easyinfra_amd.workloads import SHAPES, make_inputs


# --------------------------------------------------------------------------- router
def _brute_route(logits, k, renorm):
    T, E = logits.shape
    ids = np.zeros((T, k), dtype=np.int64)
    w = np.zeros((T, k), dtype=np.float64)
    for t in range(T):
        row = [float(v) for v in logits[t]]
        order = sorted(range(E), key=lambda e: (-row[e], e))[:k]
        m = max(row)
        ex = [math.exp(v - m) for v in row]
        tot = sum(ex)
        sel = [ex[e] for e in order]
        den = sum(sel) if renorm else tot
        ids[t] = order
        w[t] = [v / den for v in sel]
    return ids, w


@pytest.mark.parametrize("T,E,k,renorm", [(7, 8, 2, True), (9, 64, 6, False), (5, 128, 8, True), (4, 3, 3, False)])
def test_route_topk_brute_force(T, E, k, renorm):
    g = torch.Generator().manual_seed(T * E)
    logits = torch.randn(T, E, generator=g) * 3
    ids, w = oracle.route_topk(logits, k, renorm)
    bi, bw = _brute_route(logits.double().numpy(), k, renorm)
    assert np.array_equal(ids.numpy(), bi)
    np.testing.assert_allclose(w.numpy(), bw, rtol=2e-6, atol=1e-8)


def test_route_topk_matches_reference_ops_on_tie_free_inputs():
    """modeling_qwen3_moe.py:260-263 literally: softmax(fp32) -> topk -> /sum."""
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(300, 64, generator=g)
    p = torch.softmax(logits, dim=-1, dtype=torch.float32)
    rw, ri = torch.topk(p, 6, dim=-1)
    rw = rw / rw.sum(-1, keepdim=True)
    ids, w = oracle.route_topk(logits, 6, True)
    assert torch.equal(ids.long(), ri)
    torch.testing.assert_close(w, rw, rtol=1e-6, atol=1e-8)


def test_route_topk_ties_and_closed_forms():
    logits = torch.tensor([[2.0, 2.0, 1.0, 2.0], [0.0, 0.0, 0.0, 0.0]])
    ids, w = oracle.route_topk(logits, 2, True)
    assert ids.tolist() == [[0, 1], [0, 1]]
    torch.testing.assert_close(w, torch.full((2, 2), 0.5))
    # two experts, top-1 without renorm: weight = sigmoid(l0 - l1)
    l = torch.tensor([[1.3, -0.4]])
    _, w = oracle.route_topk(l, 1, False)
    assert abs(float(w[0, 0]) - 1 / (1 + math.exp(-1.7))) < 1e-6


def test_route_topk_invariants():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(200, 32, generator=g)
    ids, w = oracle.route_topk(logits, 5, True)
    assert torch.all(w[:, :-1] >= w[:, 1:])
    torch.testing.assert_close(w.sum(-1), torch.ones(200))
    assert all(len(set(r)) == 5 for r in ids.tolist())


# --------------------------------------------------------------------------- align
def _brute_align(ids, n_loc, e_lo):
    T, k = ids.shape
    flat = ids.reshape(-1)
    order = []
    counts = []
    for e in range(n_loc):
        hit = [i for i in range(T * k) if flat[i] == e + e_lo]
        counts.append(len(hit))
        order += hit
    pos = [-1] * (T * k)
    for r, i in enumerate(order):
        pos[i] = r
    return counts, order, pos


@pytest.mark.parametrize("T,k,E,e_lo,n_loc", [(13, 2, 8, 0, 8), (20, 6, 64, 0, 64), (17, 8, 128, 32, 32), (5, 3, 4, 1, 2)])
def test_align_brute_force(T, k, E, e_lo, n_loc):
    g = torch.Generator().manual_seed(T + E)
    ids = torch.rand(T, E, generator=g).argsort(1)[:, :k].numpy()
    al = oracle.align(ids, n_loc, e_lo)
    counts, order, pos = _brute_align(ids, n_loc, e_lo)
    assert al["counts"].tolist() == counts
    assert al["offsets"].tolist() == list(np.concatenate([[0], np.cumsum(counts)]))
    assert al["sorted_flat"].tolist() == order
    assert al["pos"].tolist() == pos
    assert al["sorted_tok"].tolist() == [i // k for i in order]
    assert al["sorted_slot"].tolist() == [i % k for i in order]


def test_align_matches_stable_sort_and_scatter_add():
    """moe_all2all.py:346 (with stable=True) and blocks/moe/base.py:357-359."""
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, 16, (500, 4), generator=g)
    al = oracle.align(ids.numpy(), 16, 0)
    idx = ids.view(-1).sort(stable=True).indices
    assert al["sorted_flat"].tolist() == idx.tolist()
    counts = torch.zeros(16, dtype=torch.int64).scatter_add_(0, ids.view(-1), torch.ones(2000, dtype=torch.int64))
    assert al["counts"].tolist() == counts.tolist()


def test_align_permutation_identities():
    g = torch.Generator().manual_seed(11)
    ids = torch.randint(0, 40, (333, 3), generator=g).numpy()
    al = oracle.align(ids, 32, 4)
    sf, pos = al["sorted_flat"], al["pos"]
    assert np.array_equal(pos[sf], np.arange(sf.size))
    local = (ids.reshape(-1) >= 4) & (ids.reshape(-1) < 36)
    assert np.array_equal(np.sort(sf), np.nonzero(local)[0])
    assert np.all(pos[~local] == -1)
    seg = np.repeat(np.arange(32), al["counts"])
    assert np.array_equal(ids.reshape(-1)[sf] - 4, seg)


# --------------------------------------------------------------------------- experts
def test_silu_closed_forms():
    x = torch.tensor([0.0, 1.0, -1.0, 30.0, -30.0])
    s = oracle.silu(x)
    ref = torch.tensor([0.0, 1 / (1 + math.exp(-1)), -1 / (1 + math.exp(1)), 30.0, 0.0])
    torch.testing.assert_close(s, ref, rtol=1e-6, atol=1e-6)


def test_expert_mlp_float64_loops():
    g = torch.Generator().manual_seed(5)
    M, H, I = 3, 6, 4
    x = torch.randn(M, H, generator=g)
    wgu = torch.randn(2 * I, H, generator=g)
    wd = torch.randn(H, I, generator=g)
    y = oracle.expert_mlp(x, wgu, wd)
    X, Wg, Wd = x.double().numpy(), wgu.double().numpy(), wd.double().numpy()
    ref = np.zeros((M, H))
    for m in range(M):
        h = []
        for i in range(I):
            gv = sum(X[m, j] * Wg[i, j] for j in range(H))
            uv = sum(X[m, j] * Wg[I + i, j] for j in range(H))
            h.append(gv / (1 + math.exp(-gv)) * uv)
        for o in range(H):
            ref[m, o] = sum(h[i] * Wd[o, i] for i in range(I))
    np.testing.assert_allclose(y.numpy(), ref, rtol=1e-4, atol=1e-5)


def test_expert_mlp_gate_up_halves_are_not_interchangeable():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(4, 8, generator=g)
    wgu = torch.randn(10, 8, generator=g)
    wd = torch.randn(8, 5, generator=g)
    swapped = torch.cat([wgu[5:], wgu[:5]])
    assert not torch.allclose(oracle.expert_mlp(x, wgu, wd), oracle.expert_mlp(x, swapped, wd))


# --------------------------------------------------------------------------- layer
@pytest.mark.parametrize("name", list(SHAPES))
def test_moe_forward_vs_dense_float64(name):
    inp = make_inputs(SHAPES[name], 11, device="cpu", hidden=64, inter=32)
    s = inp.shape
    a = oracle.moe_forward(inp.x, inp.logits, s.top_k, inp.w_gate_up, inp.w_down, s.renormalize,
                           inp.shared_gate_up, inp.shared_down, inp.expert_range)
    b = oracle.moe_forward_dense(inp.x, inp.logits, s.top_k, inp.w_gate_up, inp.w_down, s.renormalize,
                                 inp.shared_gate_up, inp.shared_down, inp.expert_range)
    np.testing.assert_allclose(a.double().numpy(), b.numpy(), rtol=1e-4, atol=1e-6)


def test_moe_forward_expert_parallel_decomposition():
    """Summing the EP shares of disjoint expert windows gives the whole layer."""
    inp = make_inputs(SHAPES["mixtral-8x7b"], 17, device="cpu", hidden=64, inter=32)
    s = inp.shape
    full = oracle.moe_forward(inp.x, inp.logits, 2, inp.w_gate_up, inp.w_down, True)
    parts = sum(oracle.moe_forward(inp.x, inp.logits, 2, inp.w_gate_up[lo:lo + 4], inp.w_down[lo:lo + 4], True,
                                   expert_range=(lo, lo + 4)) for lo in (0, 4))
    torch.testing.assert_close(parts, full, rtol=1e-5, atol=1e-6)


def test_moe_forward_subset_shared_and_linearity():
    inp = make_inputs(SHAPES["deepseek-v2-lite"], 9, device="cpu", hidden=64, inter=32)
    s = inp.shape
    args = (inp.x, inp.logits, s.top_k, inp.w_gate_up, inp.w_down, s.renormalize)
    full = oracle.moe_forward(*args, inp.shared_gate_up, inp.shared_down)
    sub = torch.tensor([7, 2, 5])
    part = oracle.moe_forward(*args, inp.shared_gate_up, inp.shared_down, token_subset=sub)
    torch.testing.assert_close(part, full[sub])
    no_sh = oracle.moe_forward(*args)
    torch.testing.assert_close(full, no_sh + oracle.shared_mlp(inp.x.float(), inp.shared_gate_up, inp.shared_down),
                               rtol=1e-5, atol=1e-6)
    twice = oracle.moe_forward(inp.x, inp.logits, s.top_k, inp.w_gate_up, 2 * inp.w_down, s.renormalize)
    torch.testing.assert_close(twice, 2 * no_sh, rtol=1e-5, atol=1e-6)


def test_moe_forward_no_local_expert_gives_zero_rows():
    inp = make_inputs(SHAPES["qwen3-30b-a3b-local32"], 200, device="cpu", hidden=64, inter=32)
    out, parts = oracle.moe_forward(inp.x, inp.logits, 8, inp.w_gate_up, inp.w_down, True,
                                    expert_range=(0, 32), return_parts=True)
    none_local = ~(parts["ids"] < 32).any(1)
    assert none_local.any()
    assert torch.count_nonzero(out[none_local]) == 0


# --------------------------------------------------------------------------- fp8
def test_quantize_rows_fp8_exact_values_and_rne_ties():
    # absmax 448 -> scale 1: values are quantised as themselves
    x = torch.tensor([[448.0, 1.0625, 1.1875, -2.5, 0.0, 0.013671875]])
    q, s = oracle.quantize_rows_fp8(x)
    assert float(s[0]) == 1.0
    # 1.0625 is halfway between 1.0 and 1.125 -> even mantissa (1.0);
    # 1.1875 halfway between 1.125 and 1.25 -> even (1.25); 0.013671875 = 7*2^-9 is an e4m3 subnormal
    assert q.float().tolist() == [[448.0, 1.0, 1.25, -2.5, 0.0, 0.013671875]]


def test_quantize_rows_fp8_scale_and_error_bound():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(50, 300, generator=g) * 0.02
    x[3] = 0
    q, s = oracle.quantize_rows_fp8(x)
    amax = x.abs().amax(1)
    torch.testing.assert_close(s[amax > 0], (amax / 448.0)[amax > 0])
    assert float(s[3]) == 1.0 and torch.count_nonzero(q[3].float()) == 0
    deq = q.float() * s[:, None]
    # e4m3: 3 mantissa bits -> relative error <= 2^-4 for normal values, absolute 2^-10*s below
    err = (deq - x).abs()
    bound = torch.maximum(x.abs() * 2 ** -4, (2 ** -10) * s[:, None])
    assert torch.all(err <= bound * 1.0001)
    assert torch.all(q.float().abs() <= 448)


def test_fp8_forward_with_exactly_representable_weights_matches_bf16():
    """W8A16 on weights that are already e4m3 values times their scale equals the bf16 layer."""
    inp = make_inputs(SHAPES["mixtral-8x7b"], 8, device="cpu", hidden=64, inter=32)
    qgu, sgu = oracle.quantize_weights_fp8(inp.w_gate_up.float())
    qd, sd = oracle.quantize_weights_fp8(inp.w_down.float())
    wgu = qgu.float() * sgu[..., None]
    wd = qd.float() * sd[..., None]
    a = oracle.moe_forward_fp8(inp.x, inp.logits, 2, qgu, sgu, qd, sd, True, mode="w8a16")
    b = oracle.moe_forward(inp.x, inp.logits, 2, wgu, wd, True, round_h_bf16=True)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-6)


def test_grouped_gemm_single_contract():
    g = torch.Generator().manual_seed(4)
    a = torch.randn(9, 5, generator=g)
    bs = [torch.randn(3, 5, generator=g) for _ in range(3)]
    out = oracle.grouped_gemm(a, bs, [4, 0, 5])
    torch.testing.assert_close(out[:4], a[:4] @ bs[0].T)
    torch.testing.assert_close(out[4:], a[4:] @ bs[2].T)


# --------------------------------------------------------------------------- DeepSeek-V3 gate
def _v3_gate_literal(logits, k, n_group, topk_group, bias, norm, scaling):
    """modeling_deepseek_v3.py:151-203 transcribed line by line in torch fp32 (sorted=False
    top-k calls included): the check for oracle.route_grouped_topk, not the oracle itself."""
    seq_len = logits.shape[0]
    E = logits.shape[1]
    scores = logits.float().sigmoid()
    scores_for_choice = scores.view(seq_len, -1) + bias.unsqueeze(0)
    group_scores = scores_for_choice.view(seq_len, n_group, -1).topk(2, dim=-1)[0].sum(dim=-1)
    group_idx = torch.topk(group_scores, k=topk_group, dim=-1, sorted=False)[1]
    group_mask = torch.zeros_like(group_scores)
    group_mask.scatter_(1, group_idx, 1)
    score_mask = group_mask.unsqueeze(-1).expand(seq_len, n_group, E // n_group).reshape(seq_len, -1)
    tmp_scores = scores_for_choice.masked_fill(~score_mask.bool(), 0.0)
    _, topk_idx = torch.topk(tmp_scores, k=k, dim=-1, sorted=False)
    topk_weight = scores.gather(1, topk_idx)
    if k > 1 and norm:
        topk_weight = topk_weight / (topk_weight.sum(dim=-1, keepdim=True) + 1e-20)
    return topk_idx, topk_weight * scaling


@pytest.mark.parametrize("T,E,k,ng,tg,norm,scale", [(300, 256, 8, 8, 4, True, 2.5), (200, 64, 6, 1, 1, True, 2.446),
                                                    (100, 160, 6, 10, 3, False, 1.0), (50, 512, 32, 256, 16, True, 1.5)])
def test_grouped_router_matches_reference_lines(T, E, k, ng, tg, norm, scale):
    g = torch.Generator().manual_seed(E + k)
    logits = torch.randn(T, E, generator=g) * 2
    bias = torch.randn(E, generator=g) * 0.1
    ids, w = oracle.route_grouped_topk(logits, k, ng, tg, bias, norm, scale)
    rid, rw = _v3_gate_literal(logits, k, ng, tg, bias, norm, scale)
    # the reference's order is unspecified (sorted=False): compare per token as sets, and the
    # weights matched by expert id; fp32 sigmoid vs the correctly rounded one is ~1 ulp
    for t in range(T):
        a = dict(zip(ids[t].tolist(), w[t].tolist()))
        b = dict(zip(rid[t].tolist(), rw[t].tolist()))
        assert set(a) == set(b), t
        for e in a:
            assert abs(a[e] - b[e]) <= 2e-6 * max(1.0, abs(b[e])), (t, e)


def test_grouped_router_known_answer():
    # E=8 in 4 groups of 2, keep 2 groups, k=2.  sigmoid(l) ~ [.953 .047 .622 .599 .881 .870 .269 .971];
    # group top-2 sums ~ [1.000 1.221 1.751 1.240].  Without a bias groups 2 and 3 are kept and
    # the picks are 7, 4; a -0.9 correction on expert 7 drops group 3 to ~0.34, so groups 2 and
    # 1 are kept and the picks are 4, 5.  Expert 0 (second largest sigmoid) is never picked:
    # its group is not kept.
    logits = torch.tensor([[3.0, -3.0, 0.5, 0.4, 2.0, 1.9, -1.0, 3.5]])
    s = 1 / (1 + np.exp(-logits.double().numpy()[0]))
    ids, w = oracle.route_grouped_topk(logits, 2, 4, 2, None, True, 2.0)
    assert ids.tolist() == [[7, 4]]
    np.testing.assert_allclose(w.numpy()[0], np.array([s[7], s[4]]) / (s[7] + s[4]) * 2.0, rtol=1e-6)
    bias = torch.tensor([0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, -0.9])
    ids, w = oracle.route_grouped_topk(logits, 2, 4, 2, bias, True, 2.0)
    assert ids.tolist() == [[4, 5]]
    np.testing.assert_allclose(w.numpy()[0], np.array([s[4], s[5]]) / (s[4] + s[5]) * 2.0, rtol=1e-6)
    ids, w = oracle.route_grouped_topk(logits, 2, 4, 2, bias, False, 1.0)   # no renormalisation
    np.testing.assert_allclose(w.numpy()[0], np.array([s[4], s[5]]), rtol=1e-6)


def test_grouped_router_masked_experts_score_zero():
    # Every corrected score inside the kept groups is negative, so the experts masked to 0.0
    # (masked_fill, not -inf) win, the lowest ids first; weights are their unbiased sigmoids.
    logits = torch.full((1, 8), -4.0)
    logits[0, 0] = -3.0
    bias = torch.full((8,), -0.5)
    ids, w = oracle.route_grouped_topk(logits, 3, 4, 1, bias, False, 1.0)
    # group 0 kept (largest top-2 sum); masked groups contribute experts 2, 3, 4 at 0.0
    assert ids.tolist() == [[2, 3, 4]]
    np.testing.assert_allclose(w.numpy()[0], 1 / (1 + np.exp(4.0)) * np.ones(3), rtol=1e-6)


# --------------------------------------------------------------------------- EPLB replica map
def test_eplb_default_layout_and_map_known_answer():
    from easyinfra_amd.ops import eplb_default_layout
    # 8 logical experts over 2 ranks of 5 physical slots (base.py:162-185): rank r holds its 4
    # experts and replicates the next one (mod 8): physical 0..4 -> 0 1 2 3 4, 5..9 -> 4 5 6 7 0
    phy2log, log2phy, count = eplb_default_layout(8, 2, 5)
    assert phy2log.tolist() == [[0, 1, 2, 3, 4], [4, 5, 6, 7, 0]]
    assert count.tolist() == [2, 1, 1, 1, 2, 1, 1, 1]
    assert log2phy[0].tolist() == [0, 9] and log2phy[4].tolist() == [4, 5] and log2phy[5].tolist() == [6, -1]
    # flat slot i takes replica i % count: expert 0 at slots 0, 2 -> replica 0 (physical 0),
    # expert 4 at slots 1, 3 -> replica 1 (physical 5); swapped columns flip the replicas
    ids = torch.tensor([[0, 4], [0, 4]], dtype=torch.int32)
    assert oracle.eplb_map(ids, log2phy, count).tolist() == [[0, 5], [0, 5]]
    ids = torch.tensor([[4, 0], [4, 0], [1, 7]], dtype=torch.int32)
    assert oracle.eplb_map(ids, log2phy, count).tolist() == [[4, 9], [4, 9], [1, 8]]
    assert oracle.eplb_map(torch.tensor([[-1, 8]], dtype=torch.int32), log2phy, count).tolist() == [[-1, -1]]


def test_eplb_map_invariants():
    from easyinfra_amd.ops import eplb_default_layout
    phy2log, log2phy, count = eplb_default_layout(64, 4, 20)
    g = torch.Generator().manual_seed(0)
    ids = torch.randint(0, 64, (500, 6), generator=g, dtype=torch.int32)
    phys = oracle.eplb_map(ids, log2phy, count)
    flat_p2l = phy2log.reshape(-1)
    assert torch.equal(flat_p2l[phys.long()], ids)                     # every pick keeps its logical expert
    # a replicated expert's picks alternate over its replicas with the flat slot parity
    for l in torch.nonzero(count > 1).flatten().tolist():
        sel = (ids.reshape(-1) == l).nonzero().flatten()
        got = phys.reshape(-1)[sel]
        want = log2phy[l][(sel % int(count[l])).long()]
        assert torch.equal(got, want)


# --------------------------------------------------------------------------- prologue
def _bf16_np(x64):
    """float64 -> nearest bf16 (ties to even), as float64."""
    return torch.from_numpy(np.asarray(x64, dtype=np.float64)).to(torch.float32).to(torch.bfloat16).double().numpy()


def test_prologue_matches_float64_formulation():
    g = torch.Generator().manual_seed(0)
    T, H, E = 64, 512, 8
    hid = (torch.randn(T, H, generator=g) * 2).to(torch.bfloat16)
    res = (torch.randn(T, H, generator=g) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    gw = (0.05 * torch.randn(E, H, generator=g)).to(torch.bfloat16)
    r, normed, logits = oracle.moe_prologue(hid, res, w, 1e-6, gw, logits_bf16=False)
    # residual add: exact sum rounded once to bf16
    r64 = res.double().numpy() + hid.double().numpy()
    assert np.array_equal(r.double().numpy(), _bf16_np(r64))
    # RMSNorm in float64 with the same two bf16 roundings
    rr = r.double().numpy()
    rs = 1 / np.sqrt((rr ** 2).mean(-1, keepdims=True) + 1e-6)
    n64 = _bf16_np(w.double().numpy() * _bf16_np(rr * rs))
    same = normed.double().numpy() == n64
    assert same.mean() > 0.999
    ulp = np.abs(n64) * 2.0 ** -7
    assert np.all(np.abs(normed.double().numpy() - n64) <= ulp + 1e-30)
    # fp32 logits against float64 dot products of the bf16 normed rows
    l64 = normed.double().numpy() @ gw.double().numpy().T
    np.testing.assert_allclose(logits.numpy(), l64, rtol=1e-5, atol=1e-6)


def test_prologue_rmsnorm_closed_forms():
    H = 256
    w = torch.full((H,), 0.5).to(torch.bfloat16)
    gw = torch.zeros(2, H, dtype=torch.bfloat16)
    gw[0] = 1.0
    # a constant row c: t = c / sqrt(c^2 + eps) -> +-1 for eps = 0; normed = w * sign(c)
    hid = torch.zeros(3, H, dtype=torch.bfloat16)
    res = torch.tensor([[3.0], [-0.25], [7.0]]).expand(3, H).to(torch.bfloat16).contiguous()
    _, normed, logits = oracle.moe_prologue(hid, res, w, 0.0, gw, logits_bf16=False)
    assert torch.equal(normed[0], w) and torch.equal(normed[1], -w)
    assert float(logits[0, 0]) == H * 0.5 and float(logits[0, 1]) == 0.0
    # scale invariance: doubling a row (exact in bf16) leaves the normed row unchanged
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, H, generator=g).to(torch.bfloat16)
    _, n1, _ = oracle.moe_prologue(torch.zeros_like(x), x, w, 0.0, gw)
    _, n2, _ = oracle.moe_prologue(torch.zeros_like(x), x * 2, w, 0.0, gw)
    assert torch.equal(n1, n2)


def test_prologue_bf16_logits_are_rounded_fp32_dots():
    g = torch.Generator().manual_seed(2)
    T, H, E = 32, 256, 16
    hid = torch.randn(T, H, generator=g).to(torch.bfloat16)
    res = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = torch.ones(H, dtype=torch.bfloat16)
    gw = (0.1 * torch.randn(E, H, generator=g)).to(torch.bfloat16)
    _, normed, lb = oracle.moe_prologue(hid, res, w, 1e-6, gw, logits_bf16=True)
    l64 = normed.double().numpy() @ gw.double().numpy().T
    exact = _bf16_np(l64)
    assert (lb.double().numpy() == exact).mean() > 0.99
    assert np.all(np.abs(lb.double().numpy() - exact) <= np.abs(exact) * 2.0 ** -7 + 1e-30)


# --------------------------------------------------------------------------- fp8 W8A8 pins
def _e4m3_exact_rows(rows, cols, g, log2_scale):
    """Rows of e4m3 values times 2^log2_scale[row], each row's absmax exactly 448 * 2^j: per-row
    absmax/448 quantisation gives scale 2^j and q equal to the values themselves."""
    v = (torch.randn(rows, cols, generator=g) * 60).to(torch.float8_e4m3fn).float()
    v[:, 0] = 448.0 * torch.where(torch.rand(rows, generator=g) < 0.5, -1.0, 1.0)
    return v * torch.pow(2.0, log2_scale.float())[:, None], v


def test_w8a8_gate_up_is_exact_on_representable_operands():
    """Quantisation is the identity on these operands, so W8A8 gate/up equals the float64 product
    (a dropped or doubled scale, or a transposed operand, breaks it)."""
    g = torch.Generator().manual_seed(31)
    T, H, N = 12, 256, 64
    x, xv = _e4m3_exact_rows(T, H, g, torch.randint(-12, -4, (T,), generator=g))
    w, wv = _e4m3_exact_rows(N, H, g, torch.randint(-16, -10, (N,), generator=g))
    xq, sx = oracle.quantize_rows_fp8(x)
    assert torch.equal(xq.float(), xv) and torch.equal(sx * 448, x.abs().amax(1))
    wq, sw = oracle.quantize_rows_fp8(w)
    gu = oracle.gate_up_fp8(x, wq, sw, "w8a8")
    exact = x.double() @ w.double().T
    torch.testing.assert_close(gu.double(), exact, rtol=1e-6, atol=1e-9 * float(exact.abs().max()))


def test_w8a8_gate_up_power_of_two_scale_invariance():
    """Scaling a token row by 2^j leaves its e4m3 values unchanged and scales its gate/up row by 2^j."""
    g = torch.Generator().manual_seed(32)
    x = torch.randn(6, 128, generator=g)
    w = torch.randn(40, 128, generator=g) * 0.02
    wq, sw = oracle.quantize_rows_fp8(w)
    j = torch.tensor([0, 3, -5, 7, -1, 2], dtype=torch.float32)
    xs = x * torch.pow(2.0, j)[:, None]
    q0, s0 = oracle.quantize_rows_fp8(x)
    q1, s1 = oracle.quantize_rows_fp8(xs)
    assert torch.equal(q0.float(), q1.float())
    assert torch.equal(s1, s0 * torch.pow(2.0, j))
    g0 = oracle.gate_up_fp8(x, wq, sw, "w8a8")
    g1 = oracle.gate_up_fp8(xs, wq, sw, "w8a8")
    assert torch.equal(g1, g0 * torch.pow(2.0, j)[:, None])


def test_w8a8_expert_h_quantisation_step():
    """With exact operands the only roundings left are h's: bf16 storage, then per-row e4m3.
    The oracle's expert output equals quantize(bf16(h64)) applied to the float64 down projection."""
    g = torch.Generator().manual_seed(33)
    T, H, I = 10, 128, 64
    x, _ = _e4m3_exact_rows(T, H, g, torch.randint(-8, -5, (T,), generator=g))
    wgu, _ = _e4m3_exact_rows(2 * I, H, g, torch.randint(-14, -11, (2 * I,), generator=g))
    wd, _ = _e4m3_exact_rows(H, I, g, torch.randint(-14, -11, (H,), generator=g))
    qgu, sgu = oracle.quantize_rows_fp8(wgu)
    qd, sd = oracle.quantize_rows_fp8(wd)
    y = oracle.expert_mlp_fp8(x, qgu, sgu, qd, sd, "w8a8")
    gu = x.double() @ wgu.double().T
    h64 = gu[:, :I] * torch.sigmoid(gu[:, :I]) * gu[:, I:]
    hq, sh = oracle.quantize_rows_fp8(h64.float().to(torch.bfloat16).float())
    ref = (hq.double() * sh.double()[:, None]) @ wd.double().T
    # fp32 vs float64 h can straddle an e4m3 rounding boundary for a rare element
    assert oracle.rel_l2(y, ref) <= 2e-3
    assert float(((y.double() - ref).abs() <= 1e-5 * ref.abs().max()).double().mean()) >= 0.95


def test_w8a8_five_percent_bound_is_unreachable_at_config4_quantisation():
    """Config 4's quantisation (per-channel absmax/448 e4m3 weights, per-token e4m3 activations)
    alone, with no kernel involved: rounding just x and W_gate_up to e4m3 already moves the expert
    output by more than 5e-2 rel-L2 at N(0,1) activations and N(0,0.02) weights, so W8A8 (which
    also rounds h and W_down) cannot meet 5e-2 against the bf16 layer; W8A16 can."""
    g = torch.Generator().manual_seed(4)
    T, H, I = 32, 1024, 2816
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).float()
    wgu = (torch.randn(2 * I, H, generator=g) * 0.02).to(torch.bfloat16).float()
    wd = (torch.randn(H, I, generator=g) * 0.02).to(torch.bfloat16).float()
    qgu, sgu = oracle.quantize_rows_fp8(wgu)
    qd, sd = oracle.quantize_rows_fp8(wd)
    ref = oracle.expert_mlp(x, wgu, wd)
    gu_only = oracle.gate_up_fp8(x, qgu, sgu, "w8a8")
    y_gu_only = (oracle.silu(gu_only[:, :I]) * gu_only[:, I:]) @ wd.T
    full = oracle.expert_mlp_fp8(x, qgu, sgu, qd, sd, "w8a8")
    w8a16 = oracle.expert_mlp_fp8(x, qgu, sgu, qd, sd, "w8a16")
    assert oracle.rel_l2(y_gu_only, ref) > 5e-2
    assert 5e-2 < oracle.rel_l2(full, ref) < 8e-2
    assert oracle.rel_l2(w8a16, ref) < 5e-2
