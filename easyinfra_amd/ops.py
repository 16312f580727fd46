"""Torch-facing wrappers of the HIP kernels (one per C-ABI entry point).

Tensors must already live on the GPU; each call enqueues on the current torch
stream and returns fresh output tensors (the reference's ``new_empty`` outputs,
fused_moe.py:444, 464).  Nothing here synchronises the device or falls back to
PyTorch math: a missing library or an unsupported shape raises.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import call

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float8_e4m3fn: _lib.FP8}


def _dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


def _req(t: torch.Tensor, name: str, dtype=None, dim=None):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if dim is not None and t.dim() != dim:
        raise ValueError(f"{name} must be {dim}-D, got {tuple(t.shape)}")


def _req_shape(t: torch.Tensor, name: str, shape: Tuple[int, ...], dtype=torch.float32):
    """A tensor whose extent the kernels assume without reading it (scales, shared weights):
    refuse anything but exactly ``shape`` before a launch could read past it."""
    _req(t, name, dtype)
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def _req_rows(t: torch.Tensor, name: str, rows: int):
    if t.shape[0] < rows:
        raise ValueError(f"{name} has {t.shape[0]} rows, max_rows={rows} needs at least that many")


def router_topk(logits: torch.Tensor, top_k: int, renormalize: bool = True) -> Tuple[torch.Tensor, torch.Tensor]:
    """modeling_qwen3_moe.py:255-266 -> (ids int32 [T,k], weights fp32 [T,k])."""
    _req(logits, "logits", torch.float32, 2)
    T, E = logits.shape
    ids = torch.empty(T, top_k, dtype=torch.int32, device=logits.device)
    w = torch.empty(T, top_k, dtype=torch.float32, device=logits.device)
    call("eimoe_router_topk", logits.data_ptr(), T, E, top_k, int(renormalize), ids.data_ptr(), w.data_ptr(),
         _stream(logits))
    return ids, w


def moe_prologue(hidden: torch.Tensor, residual: torch.Tensor, norm_w: torch.Tensor, eps: float,
                 gate_w: torch.Tensor, logits_bf16: bool = True, residual_out: Optional[torch.Tensor] = None,
                 workspace: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Residual add, post-attention RMSNorm and router logits in one pass
    (moe_all2all.py:329-336, base_rmsnorm.py:6-12, base_linear.py:28-36)
    -> (residual_out [T,H] bf16, normed [T,H] bf16, logits [T,E] fp32).  ``logits_bf16`` rounds the
    logits to bf16 values (a bf16 gate F.linear: Qwen3, Mixtral); False keeps fp32 (DeepSeek-V3)."""
    _req(hidden, "hidden", torch.bfloat16, 2)
    _req(residual, "residual", torch.bfloat16, 2)
    _req(norm_w, "norm_w", torch.bfloat16, 1)
    _req(gate_w, "gate_w", torch.bfloat16, 2)
    T, H = hidden.shape
    E = gate_w.shape[0]
    if tuple(residual.shape) != (T, H) or norm_w.numel() != H or gate_w.shape[1] != H:
        raise ValueError(f"shapes: hidden {tuple(hidden.shape)}, residual {tuple(residual.shape)}, "
                         f"norm_w {tuple(norm_w.shape)}, gate_w {tuple(gate_w.shape)}")
    dev = hidden.device
    res_out = torch.empty_like(residual) if residual_out is None else residual_out
    normed = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    logits = torch.empty(T, E, dtype=torch.float32, device=dev)
    need = moe_prologue_workspace_bytes(T, H, E)
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    call("eimoe_moe_prologue", hidden.data_ptr(), residual.data_ptr(), norm_w.data_ptr(), float(eps),
         gate_w.data_ptr(), T, H, E, _lib.LOGITS_BF16 if logits_bf16 else 0, res_out.data_ptr(), normed.data_ptr(),
         logits.data_ptr(), _ptr(workspace), 0 if workspace is None else workspace.numel(), _stream(hidden))
    return res_out, normed, logits


def moe_prologue_workspace_bytes(T: int, H: int, E: int) -> int:
    """Workspace bytes ``moe_prologue`` needs at these sizes (0 when the router is dotted in the
    same pass; else the router GEMM's segment offsets and K-split planes)."""
    return int(_lib.lib().eimoe_moe_prologue_workspace_bytes(T, H, E))


def router_grouped_topk(logits: torch.Tensor, top_k: int, n_group: int = 1, topk_group: int = 1,
                        bias: Optional[torch.Tensor] = None, renormalize: bool = True,
                        scaling: float = 1.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """DeepseekV3MoEGate.forward, "noaux_tc" (modeling_deepseek_v3.py:151-203) from the logits on
    -> (ids int32 [T,k], weights fp32 [T,k])."""
    _req(logits, "logits", torch.float32, 2)
    T, E = logits.shape
    if bias is not None:
        _req(bias, "bias", torch.float32, 1)
        if bias.numel() != E:
            raise ValueError(f"bias has {bias.numel()} entries, logits {E} experts")
    ids = torch.empty(T, top_k, dtype=torch.int32, device=logits.device)
    w = torch.empty(T, top_k, dtype=torch.float32, device=logits.device)
    call("eimoe_router_grouped_topk", logits.data_ptr(), T, E, top_k, n_group, topk_group, _ptr(bias),
         int(renormalize), float(scaling), ids.data_ptr(), w.data_ptr(), _stream(logits))
    return ids, w


def eplb_default_layout(num_logical: int, ep_size: int, num_physical: int):
    """The default replica layout of _MoeBlock (generation/blocks/moe/base.py:162-185), built on
    the host: each of ``ep_size`` ranks holds ``num_physical`` physical experts, its share of
    the logical experts followed by replicas of the next ones.  Returns (phy2log [ep, P],
    log2phy [L, max_replicas] (-1 padded), replica_count [L]), int32 CPU tensors."""
    base_n = num_logical // ep_size
    if base_n * ep_size != num_logical or num_physical < base_n:
        raise ValueError(f"{num_logical} logical experts over ep={ep_size} with {num_physical} physical per rank")
    base = torch.arange(base_n * ep_size).view(ep_size, base_n)
    tail = torch.arange(1, num_physical - base_n + 1)[None, :] + base[:, -1:]
    phy2log = torch.cat([base, tail], dim=-1) % num_logical
    flat = phy2log.reshape(-1)
    count = torch.bincount(flat, minlength=num_logical)
    log2phy = torch.full((num_logical, int(count.max())), -1, dtype=torch.long)
    fill = torch.zeros(num_logical, dtype=torch.long)
    for p, l in enumerate(flat.tolist()):
        log2phy[l, fill[l]] = p
        fill[l] += 1
    return phy2log.to(torch.int32), log2phy.to(torch.int32), count.to(torch.int32)


def eplb_map(topk_ids: torch.Tensor, log2phy: torch.Tensor, replica_count: torch.Tensor,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Logical -> physical expert ids (base.py:40-64): replica (t*k + slot) mod count."""
    _req(topk_ids, "topk_ids", torch.int32, 2)
    _req(log2phy, "log2phy", torch.int32, 2)
    _req(replica_count, "replica_count", torch.int32, 1)
    T, k = topk_ids.shape
    out = torch.empty_like(topk_ids) if out is None else out
    call("eimoe_eplb_map", topk_ids.data_ptr(), T, k, log2phy.data_ptr(), log2phy.shape[0], log2phy.shape[1],
         replica_count.data_ptr(), out.data_ptr(), _stream(topk_ids))
    return out


def align(topk_ids: torch.Tensor, n_local: int, e_lo: int = 0, one_workgroup: bool = False) -> dict:
    """Counts/offsets/stable permutation (blocks/moe/base.py:343-364, moe_all2all.py:346-348).
    Large batches sort over many workgroups (a small workspace); ``one_workgroup`` forces the
    single-workgroup kernel (the same result)."""
    _req(topk_ids, "topk_ids", torch.int32, 2)
    T, k = topk_ids.shape
    dev = topk_ids.device
    A = T * k
    need = 0 if one_workgroup else int(_lib.lib().eimoe_align_workspace_bytes(T, k, n_local))
    ws = torch.empty(need, dtype=torch.uint8, device=dev) if need else None
    out = {
        "counts": torch.empty(n_local, dtype=torch.int32, device=dev),
        "offsets": torch.empty(n_local + 1, dtype=torch.int32, device=dev),
        "sorted_flat": torch.empty(A, dtype=torch.int32, device=dev),
        "sorted_tok": torch.empty(A, dtype=torch.int32, device=dev),
        "pos": torch.empty(A, dtype=torch.int32, device=dev),
    }
    call("eimoe_align", topk_ids.data_ptr(), T, k, e_lo, n_local, out["counts"].data_ptr(),
         out["offsets"].data_ptr(), out["sorted_flat"].data_ptr(), out["sorted_tok"].data_ptr(),
         out["pos"].data_ptr(), _ptr(ws), need, _stream(topk_ids))
    return out


def route_align(logits: torch.Tensor, top_k: int, n_local: int, e_lo: int = 0,
                renormalize: bool = True) -> Tuple[torch.Tensor, torch.Tensor, dict]:
    """router_topk then align in one call (one launch for small batches) -> (ids, weights, align dict)."""
    _req(logits, "logits", torch.float32, 2)
    T, E = logits.shape
    dev = logits.device
    A = T * top_k
    ids = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    w = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    out = {
        "counts": torch.empty(n_local, dtype=torch.int32, device=dev),
        "offsets": torch.empty(n_local + 1, dtype=torch.int32, device=dev),
        "sorted_flat": torch.empty(A, dtype=torch.int32, device=dev),
        "sorted_tok": torch.empty(A, dtype=torch.int32, device=dev),
        "pos": torch.empty(A, dtype=torch.int32, device=dev),
    }
    call("eimoe_route_align", logits.data_ptr(), T, E, top_k, int(renormalize), e_lo, n_local, ids.data_ptr(),
         w.data_ptr(), out["counts"].data_ptr(), out["offsets"].data_ptr(), out["sorted_flat"].data_ptr(),
         out["sorted_tok"].data_ptr(), out["pos"].data_ptr(), _stream(logits))
    return ids, w, out


def counts_to_offsets(counts: torch.Tensor) -> torch.Tensor:
    _req(counts, "counts", torch.int32, 1)
    off = torch.empty(counts.numel() + 1, dtype=torch.int32, device=counts.device)
    call("eimoe_counts_to_offsets", counts.data_ptr(), counts.numel(), off.data_ptr(), _stream(counts))
    return off


def gather(x: torch.Tensor, rows: torch.Tensor, num_rows: torch.Tensor, max_rows: int) -> torch.Tensor:
    """xs[r] = x[rows[r]] for r < num_rows (a 1-element device tensor), moe_all2all.py:351."""
    _req(x, "x", (torch.float32, torch.bfloat16), 2)
    _req(rows, "rows", torch.int32)
    xs = torch.empty(max_rows, x.shape[1], dtype=x.dtype, device=x.device)
    call("eimoe_gather", x.data_ptr(), _dt(x), x.shape[1], rows.data_ptr(), num_rows.data_ptr(), max_rows,
         xs.data_ptr(), _stream(x))
    return xs


def gemm_gate_up_silu(a: torch.Tensor, w_gate_up: torch.Tensor, seg_offsets: torch.Tensor, max_rows: int,
                      a_rows: Optional[torch.Tensor] = None, w_scale: Optional[torch.Tensor] = None,
                      e_mod: Optional[int] = None, tile: int = 0) -> torch.Tensor:
    """fused_moe.py:445-459: h = silu(a.Wg^T) * (a.Wu^T) per segment -> bf16 [max_rows, I]
    (fp32 a and weights: the fp32 MFMA, fp32 h)."""
    f32 = w_gate_up.dtype == torch.float32
    _req(a, "a", torch.float32 if f32 else torch.bfloat16, 2)
    _req(w_gate_up, "w_gate_up", (torch.bfloat16, torch.float8_e4m3fn, torch.float32), 3)
    _req(seg_offsets, "seg_offsets", torch.int32, 1)
    E, I2, H = w_gate_up.shape
    I = I2 // 2
    if a.shape[1] != H:
        raise ValueError(f"a has {a.shape[1]} columns, weights expect H={H}")
    if a_rows is not None:
        _req(a_rows, "a_rows", torch.int32)
        _req_rows(a_rows, "a_rows", max_rows)
    else:
        _req_rows(a, "a", max_rows)
    if (w_scale is not None) != (w_gate_up.dtype == torch.float8_e4m3fn):
        raise ValueError("fp8 weights need w_scale [E, 2I]; bf16 weights take none")
    if w_scale is not None:
        _req_shape(w_scale, "w_scale", (E, I2))
    h = torch.empty(max_rows, I, dtype=torch.float32 if f32 else torch.bfloat16, device=a.device)
    call("eimoe_gemm_gate_up_silu", a.data_ptr(), _ptr(a_rows), a.shape[0], a.stride(0), w_gate_up.data_ptr(),
         _dt(w_gate_up),
         _ptr(w_scale), H, I, seg_offsets.data_ptr(), seg_offsets.numel() - 1, e_mod or E, max_rows, h.data_ptr(),
         tile, _stream(a))
    return h


def gemm_down(h: torch.Tensor, w_down: torch.Tensor, seg_offsets: torch.Tensor, max_rows: int,
              out_dtype=torch.float32, k_split: int = 1, w_scale: Optional[torch.Tensor] = None,
              e_mod: Optional[int] = None, tile: int = 0) -> torch.Tensor:
    """fused_moe.py:463-476: y = h . Wd^T per segment -> [k_split, max_rows, H] partial planes
    (fp32 h and weights: the fp32 MFMA, fp32 y)."""
    f32 = w_down.dtype == torch.float32
    _req(h, "h", torch.float32 if f32 else torch.bfloat16, 2)
    _req(w_down, "w_down", (torch.bfloat16, torch.float8_e4m3fn, torch.float32), 3)
    if f32 and out_dtype != torch.float32:
        raise TypeError("fp32 weights write fp32 y")
    _req(seg_offsets, "seg_offsets", torch.int32, 1)
    E, H, I = w_down.shape
    if h.shape[1] != I:
        raise ValueError(f"h has {h.shape[1]} columns, weights expect I={I}")
    _req_rows(h, "h", max_rows)
    if (w_scale is not None) != (w_down.dtype == torch.float8_e4m3fn):
        raise ValueError("fp8 weights need w_scale [E, H]; bf16 weights take none")
    if w_scale is not None:
        _req_shape(w_scale, "w_scale", (E, H))
    y = torch.empty(k_split, max_rows, H, dtype=out_dtype, device=h.device)
    call("eimoe_gemm_down", h.data_ptr(), I, w_down.data_ptr(), _dt(w_down), _ptr(w_scale), H,
         seg_offsets.data_ptr(), seg_offsets.numel() - 1, e_mod or E, max_rows, y.data_ptr(), _dt(y), k_split, tile,
         _stream(h))
    return y


def gemm_gate_up_silu_w8a8(aq: torch.Tensor, a_scale: torch.Tensor, w_gate_up: torch.Tensor, w_scale: torch.Tensor,
                           seg_offsets: torch.Tensor, max_rows: int, a_rows: Optional[torch.Tensor] = None,
                           e_mod: Optional[int] = None, tile: int = 0) -> torch.Tensor:
    """W8A8 gate/up: fp8 activations (per-row scales) x fp8 weights (per-channel scales), fp8 MFMA,
    silu(g)*u -> bf16 [max_rows, I]."""
    _req(aq, "aq", torch.float8_e4m3fn, 2)
    _req(a_scale, "a_scale", torch.float32)
    _req(w_gate_up, "w_gate_up", torch.float8_e4m3fn, 3)
    _req(w_scale, "w_scale", torch.float32)
    _req(seg_offsets, "seg_offsets", torch.int32, 1)
    E, I2, H = w_gate_up.shape
    I = I2 // 2
    if aq.shape[1] != H:
        raise ValueError(f"aq has {aq.shape[1]} columns, weights expect H={H}")
    _req_shape(a_scale, "a_scale", (aq.shape[0],))
    _req_shape(w_scale, "w_scale", (E, I2))
    if a_rows is not None:
        _req(a_rows, "a_rows", torch.int32)
        _req_rows(a_rows, "a_rows", max_rows)
    else:
        _req_rows(aq, "aq", max_rows)
    h = torch.empty(max_rows, I, dtype=torch.bfloat16, device=aq.device)
    call("eimoe_gemm_gate_up_silu_w8a8", aq.data_ptr(), a_scale.data_ptr(), _ptr(a_rows), aq.shape[0], aq.stride(0),
         w_gate_up.data_ptr(), w_scale.data_ptr(), H, I, seg_offsets.data_ptr(), seg_offsets.numel() - 1, e_mod or E,
         max_rows, h.data_ptr(), tile, _stream(aq))
    return h


def gemm_down_w8a8(hq: torch.Tensor, h_scale: torch.Tensor, w_down: torch.Tensor, w_scale: torch.Tensor,
                   seg_offsets: torch.Tensor, max_rows: int, out_dtype=torch.float32, k_split: int = 1,
                   e_mod: Optional[int] = None, tile: int = 0) -> torch.Tensor:
    """W8A8 down: y = (hq . Wq^T) * h_scale[row] * w_scale[col] -> [k_split, max_rows, H]."""
    _req(hq, "hq", torch.float8_e4m3fn, 2)
    _req(h_scale, "h_scale", torch.float32)
    _req(w_down, "w_down", torch.float8_e4m3fn, 3)
    _req(w_scale, "w_scale", torch.float32)
    _req(seg_offsets, "seg_offsets", torch.int32, 1)
    E, H, I = w_down.shape
    if hq.shape[1] != I:
        raise ValueError(f"hq has {hq.shape[1]} columns, weights expect I={I}")
    _req_rows(hq, "hq", max_rows)
    if h_scale.dim() != 1 or h_scale.shape[0] < max_rows:
        raise ValueError(f"h_scale must be 1-D with at least max_rows={max_rows} entries, got {tuple(h_scale.shape)}")
    _req_shape(w_scale, "w_scale", (E, H))
    y = torch.empty(k_split, max_rows, H, dtype=out_dtype, device=hq.device)
    call("eimoe_gemm_down_w8a8", hq.data_ptr(), h_scale.data_ptr(), I, w_down.data_ptr(), w_scale.data_ptr(), H,
         seg_offsets.data_ptr(), seg_offsets.numel() - 1, e_mod or E, max_rows, y.data_ptr(), _dt(y), k_split, tile,
         _stream(hq))
    return y


def grouped_gemm(a: torch.Tensor, b: torch.Tensor, seg_offsets: torch.Tensor, max_rows: int,
                 out_dtype=torch.bfloat16, a_rows: Optional[torch.Tensor] = None,
                 b_scale: Optional[torch.Tensor] = None, e_mod: Optional[int] = None, tile: int = 0) -> torch.Tensor:
    """single_group_gemm_moe.py:76-91: c[rows_s] = a[rows_s] . b[s % e_mod]^T, b packed [E,N,K]
    (fp32 a and b: the fp32 MFMA, fp32 c)."""
    f32 = b.dtype == torch.float32
    _req(a, "a", torch.float32 if f32 else torch.bfloat16, 2)
    _req(b, "b", (torch.bfloat16, torch.float8_e4m3fn, torch.float32), 3)
    if f32:
        out_dtype = torch.float32
    _req(seg_offsets, "seg_offsets", torch.int32, 1)
    E, N, K = b.shape
    if a.shape[1] != K:
        raise ValueError(f"a has {a.shape[1]} columns, b expects K={K}")
    if a_rows is not None:
        _req(a_rows, "a_rows", torch.int32)
        _req_rows(a_rows, "a_rows", max_rows)
    else:
        _req_rows(a, "a", max_rows)
    if (b_scale is not None) != (b.dtype == torch.float8_e4m3fn):
        raise ValueError("fp8 b needs b_scale [E, N]; bf16 b takes none")
    if b_scale is not None:
        _req_shape(b_scale, "b_scale", (E, N))
    c = torch.empty(max_rows, N, dtype=out_dtype, device=a.device)
    call("eimoe_grouped_gemm", a.data_ptr(), _ptr(a_rows), a.shape[0], a.stride(0), b.data_ptr(), _dt(b),
         _ptr(b_scale),
         N * K, N, K, seg_offsets.data_ptr(), seg_offsets.numel() - 1, e_mod or E, max_rows, c.data_ptr(), _dt(c),
         tile, _stream(a))
    return c


def combine(y: torch.Tensor, pos: torch.Tensor, topk_weights: torch.Tensor, shared_y: Optional[torch.Tensor] = None,
            out_dtype=torch.bfloat16) -> torch.Tensor:
    """moe_all2all.py:291-307 (+ shared-expert add): out[t] = sum_j w[t,j] * sum_s y[s][pos[t,j]]."""
    if y.dim() == 2:
        y = y.unsqueeze(0)
    _req(y, "y", (torch.float32, torch.bfloat16), 3)
    _req(topk_weights, "topk_weights", torch.float32, 2)
    _req(pos, "pos", torch.int32)
    T, k = topk_weights.shape
    n_split, rows, H = y.shape
    if pos.numel() != T * k:
        raise ValueError(f"pos has {pos.numel()} entries, topk_weights {T}x{k}")
    if shared_y is not None:
        _req(shared_y, "shared_y", (torch.float32, torch.bfloat16), 2)
        if tuple(shared_y.shape) != (T, H):
            raise ValueError(f"shared_y must be [{T}, {H}], got {tuple(shared_y.shape)}")
    out = torch.empty(T, H, dtype=out_dtype, device=y.device)
    call("eimoe_combine", y.data_ptr(), _dt(y), n_split, rows * H, pos.data_ptr(), topk_weights.data_ptr(), T, k, H,
         _ptr(shared_y), _dt(shared_y) if shared_y is not None else 0, out.data_ptr(), _dt(out), _stream(y))
    return out


def quantize_rows_fp8(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row absmax/448 scale and e4m3fn values; rows = all leading dims."""
    _req(x, "x", (torch.float32, torch.bfloat16))
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device)
    call("eimoe_quantize_rows_fp8", x.data_ptr(), _dt(x), rows, cols, q.data_ptr(), s.data_ptr(), _stream(x))
    return q, s


def quantize_weights_fp8(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Expert weights [E,N,K] -> (e4m3fn [E,N,K], per-output-channel scales [E,N])."""
    return quantize_rows_fp8(w)


def release_streams() -> None:
    """Release this thread's second stream (shared experts) and its events; the next fused_moe call
    with shared experts creates them again."""
    call("eimoe_release_streams")


def fused_moe_workspace_bytes(T, H, I, E, k, n_local, shared_inter=0, out_dtype=torch.bfloat16, flags=0) -> int:
    return int(_lib.lib().eimoe_fused_moe_workspace_bytes(T, H, I, E, k, n_local, shared_inter,
                                                           _DT[out_dtype], flags))


def fused_moe_down_split(T, H, I, E, k, n_local, shared_inter=0, out_dtype=torch.bfloat16, flags=0) -> int:
    """The down projection's K split fused_moe picks for this layer (its fp32 partial planes)."""
    return int(_lib.lib().eimoe_fused_moe_down_split(T, H, I, E, k, n_local, shared_inter, _DT[out_dtype], flags))


def fused_moe(hidden_states: torch.Tensor, router_logits: torch.Tensor, top_k: int, w_gate_up: torch.Tensor,
              w_down: torch.Tensor, *, renormalize: bool = True, shared_gate_up: Optional[torch.Tensor] = None,
              shared_down: Optional[torch.Tensor] = None, expert_range: Optional[Sequence[int]] = None,
              w_scales: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, out_dtype=None, y_fp32: bool = False,
              w8a8: bool = False, h_split: bool = False, workspace: Optional[torch.Tensor] = None,
              return_routing: bool = False,
              scoring_func: str = "softmax", n_group: int = 1, topk_group: int = 1,
              e_score_correction_bias: Optional[torch.Tensor] = None, routed_scaling_factor: float = 1.0,
              routing: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, num_experts: Optional[int] = None):
    """The MoE layer: (hidden_states [T,H], router_logits [T,E], top_k) -> combined output [T,H].

    Reproduces MoeAll2AllBlock's stages at ep=1 (moe_all2all.py:85-95) with
    FusedMoE.forward_ep (fused_moe.py:106-156) as the expert step:
    route (softmax, top-k, optional renorm) -> align -> gate/up + SiLU*mul ->
    down -> weighted combine (+ shared experts, weight 1).

    ``expert_range=(lo, hi)``: only experts [lo, hi) of the router's E are resident
    (one GPU's EP share); ``w_gate_up``/``w_down`` hold exactly those.  Tokens with
    no resident expert produce zero rows.
    ``w_scales=(s_gate_up [E,2I], s_down [E,H])`` marks fp8-e4m3 weights: bf16 activations on
    the bf16 MFMA (W8A16), or with ``w8a8=True`` activations quantised per token / per row
    and both GEMMs on the fp8 MFMA (W8A8).
    fp32 hidden states with fp32 weights run the fp32 layer (fp32 MFMA, fp32 h and y: the
    reference's fp32 F.linear path, native_moe.py:56-103); fp32 hidden states with bf16 or fp8
    weights are refused rather than rounded.
    The per-assignment expert outputs are kept in fp32 and summed by the combine in fp32 with one
    rounding to ``out_dtype`` (``y_fp32`` is accepted for compatibility and has no effect).
    ``h_split=True`` is the precise mode: h = silu(g)*u is kept as a pair of bf16 terms (hi + lo)
    and the down projection runs once per term, so h carries ~16 significant bits instead of 8
    (twice the down projection's time; per-assignment outputs in fp32).
    ``scoring_func="sigmoid"`` routes with the DeepSeek-V3 gate (``router_grouped_topk``:
    ``n_group``, ``topk_group``, ``e_score_correction_bias``, ``routed_scaling_factor``,
    ``renormalize`` as norm_topk_prob) instead of softmax top-k.  ``routing=(ids int32 [T,k],
    weights fp32 [T,k])`` skips the router altogether (``router_logits`` may then be None, with
    ``num_experts`` giving E when it is not the top of ``expert_range``).
    """
    x = hidden_states
    f32 = w_gate_up.dtype == torch.float32
    if x.dtype == torch.float32 and not f32:
        raise TypeError("fp32 hidden_states need fp32 weights (the fp32 layer); cast the hidden states to bf16 "
                        "explicitly to run them on bf16 or fp8 weights")
    _req(x, "hidden_states", torch.float32 if f32 else torch.bfloat16, 2)
    if scoring_func not in ("softmax", "sigmoid"):
        raise ValueError(f"scoring_func {scoring_func!r}: 'softmax' or 'sigmoid'")
    if scoring_func == "sigmoid" and routing is None:
        routing = router_grouped_topk(router_logits, top_k, n_group, topk_group, e_score_correction_bias,
                                      renormalize, routed_scaling_factor)
    if routing is None or router_logits is not None:
        _req(router_logits, "router_logits", torch.float32, 2)
    _req(w_gate_up, "w_gate_up", (torch.bfloat16, torch.float8_e4m3fn, torch.float32), 3)
    _req(w_down, "w_down", (w_gate_up.dtype, torch.float8_e4m3fn) if not f32 else torch.float32, 3)
    T, H = x.shape
    n_local, I2, H2 = w_gate_up.shape
    if router_logits is not None:
        E = router_logits.shape[1]
    else:
        E = num_experts or (expert_range[1] if expert_range is not None else n_local)
    I = I2 // 2
    if H2 != H or tuple(w_down.shape) != (n_local, H, I):
        raise ValueError(f"weight shapes {tuple(w_gate_up.shape)}/{tuple(w_down.shape)} do not match H={H}")
    lo, hi = expert_range if expert_range is not None else (0, E)
    if hi - lo != n_local:
        raise ValueError(f"expert_range {lo, hi} holds {hi - lo} experts, weights hold {n_local}")
    fp8 = w_gate_up.dtype == torch.float8_e4m3fn
    if fp8 != (w_down.dtype == torch.float8_e4m3fn) or fp8 != (w_scales is not None):
        raise ValueError("fp8 weights need both tensors in e4m3fn and w_scales=(s_gate_up, s_down)")
    if fp8:
        _req_shape(w_scales[0], "w_scales[0] (gate/up)", (n_local, I2))
        _req_shape(w_scales[1], "w_scales[1] (down)", (n_local, H))
    out_dtype = out_dtype or hidden_states.dtype
    Is = 0
    if (shared_gate_up is None) != (shared_down is None):
        raise ValueError("shared experts need both shared_gate_up [2*Is, H] and shared_down [H, Is]")
    if shared_gate_up is not None:
        sh_dt = torch.float32 if f32 else torch.bfloat16
        _req(shared_down, "shared_down", sh_dt, 2)
        Is = shared_down.shape[1]
        _req_shape(shared_gate_up, "shared_gate_up", (2 * Is, H), sh_dt)
        _req_shape(shared_down, "shared_down", (H, Is), sh_dt)
    if w8a8 and not fp8:
        raise ValueError("w8a8 needs fp8 weights and w_scales")
    if w8a8 and h_split:
        raise ValueError("h_split keeps h as bf16 terms; w8a8 quantises it to fp8")
    flags = (_lib.RENORMALIZE if renormalize else 0) | (_lib.Y_F32 if y_fp32 else 0) | (_lib.W8A8 if w8a8 else 0)
    flags |= _lib.H_SPLIT if h_split else 0
    if f32:
        if w8a8 or h_split:
            raise ValueError("the fp32 layer keeps h in fp32: no w8a8 or h_split")
        flags |= _lib.FP32
    if routing is not None:
        ids_in, w_in = routing
        _req(ids_in, "routing ids", torch.int32, 2)
        _req(w_in, "routing weights", torch.float32, 2)
        if tuple(ids_in.shape) != (T, top_k) or tuple(w_in.shape) != (T, top_k):
            raise ValueError(f"routing tensors must be [T={T}, k={top_k}]")
        flags |= _lib.ROUTING_IN
    need = fused_moe_workspace_bytes(T, H, I, E, top_k, n_local, Is, out_dtype, flags)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    out = torch.empty(T, H, dtype=out_dtype, device=x.device)
    ids = w = None
    if routing is not None:
        ids, w = routing
    elif return_routing:
        ids = torch.empty(T, top_k, dtype=torch.int32, device=x.device)
        w = torch.empty(T, top_k, dtype=torch.float32, device=x.device)
    s_gu, s_d = w_scales if fp8 else (None, None)
    call("eimoe_fused_moe", x.data_ptr(), _ptr(router_logits), T, H, I, E, top_k, w_gate_up.data_ptr(),
         w_down.data_ptr(), _dt(w_gate_up), _ptr(s_gu), _ptr(s_d), lo, n_local, _ptr(shared_gate_up),
         _ptr(shared_down), Is, flags, out.data_ptr(), _DT[out_dtype], workspace.data_ptr(), workspace.numel(),
         _ptr(ids), _ptr(w), _stream(x))
    if return_routing:
        return out, ids, w
    return out
