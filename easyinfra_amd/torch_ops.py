"""torch.ops registration of the grouped GEMM for the reference's native op point.

EasyInfra loads ``*.so`` op libraries and calls
``torch.ops.ops.<impl>_grouped_gemm_single(A, B_list, block_sizes)``
(easyinfra/__init__.py:7-20, single_group_gemm_moe.py:53-91): ``A[M,K]`` rows in
contiguous blocks, ``B_list`` one ``[N,K]`` nn.Linear weight per block,
``out[rows_i] = A[rows_i] @ B_i^T``.  Importing this module registers
``torch.ops.ops.hip_grouped_gemm_single`` with that schema, backed by the HIP
grouped GEMM.  The weights are read where they lie, through a device table of
per-expert pointers: the reference's list holds its experts' Parameters repeated
ep_size times (single_group_gemm_moe.py:73-76, 89), so only the first period goes
into the table and the blocks index it modulo its length.  No weight is copied.
"""
from __future__ import annotations

from typing import Dict, List, Tuple

import torch

from . import _lib, ops
from ._lib import call

_LIB = torch.library.Library("ops", "FRAGMENT")
_LIB.define("hip_grouped_gemm_single(Tensor A, Tensor[] B_list, int[] block_sizes) -> Tensor")

# device pointer tables, keyed on (device index, the weights' addresses); a few bytes each
_PTR_TABLES: Dict[Tuple[int, Tuple[int, ...]], torch.Tensor] = {}
_MAX_TABLES = 256


def _period(b_list: List[torch.Tensor]) -> int:
    """Shortest p with b_list[i] the same tensor memory as b_list[i % p] for every i."""
    n = len(b_list)
    ptrs = [b.data_ptr() for b in b_list]
    for p in range(1, n + 1):
        if n % p == 0 and all(ptrs[i] == ptrs[i % p] for i in range(n)):
            return p
    return n


def _to_device(values, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """A small host list on the device without blocking the host: staged in pinned memory and
    copied on the current stream (the caching host allocator keeps the staging block until the
    copy has run)."""
    return torch.tensor(values, dtype=dtype, pin_memory=True).to(device, non_blocking=True)


def _ptr_table(b_list: List[torch.Tensor], device: torch.device) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           tuple(b.data_ptr() for b in b_list))
    t = _PTR_TABLES.get(key)
    if t is None:
        if len(_PTR_TABLES) >= _MAX_TABLES:
            _PTR_TABLES.pop(next(iter(_PTR_TABLES)))
        t = _to_device(list(key[1]), torch.int64, device)
        _PTR_TABLES[key] = t
    # A cached table may be read on a stream other than the one it was made on: mark every use, so
    # that once evicted its memory is not handed out again before the kernels reading it have run.
    t.record_stream(torch.cuda.current_stream(device))
    return t


def hip_grouped_gemm_single(A: torch.Tensor, B_list: List[torch.Tensor], block_sizes: List[int]) -> torch.Tensor:
    if len(B_list) != len(block_sizes):
        raise ValueError(f"{len(B_list)} weights for {len(block_sizes)} blocks")
    if not B_list:
        raise ValueError("empty B_list")
    M = int(sum(block_sizes))
    if M != A.shape[0]:
        raise ValueError(f"block sizes sum to {M}, A has {A.shape[0]} rows")
    A = A.contiguous()
    ops._req(A, "A", torch.bfloat16, 2)
    N, K = B_list[0].shape
    for i, b in enumerate(B_list):
        ops._req(b, f"B_list[{i}]", torch.bfloat16, 2)
        if tuple(b.shape) != (N, K) or b.device != A.device:
            raise ValueError(f"B_list[{i}] is {tuple(b.shape)} on {b.device}, expected ({N}, {K}) on {A.device}")
    if K != A.shape[1]:
        raise ValueError(f"A has {A.shape[1]} columns, the weights K={K}")
    p = _period(B_list)
    table = _ptr_table(B_list[:p], A.device)
    bounds = [0]
    for b in block_sizes:
        bounds.append(bounds[-1] + int(b))
    off = _to_device(bounds, torch.int32, A.device)
    c = torch.empty(M, N, dtype=A.dtype, device=A.device)
    call("eimoe_grouped_gemm_ptrs", A.data_ptr(), None, A.shape[0], A.stride(0), table.data_ptr(), p, N, K,
         off.data_ptr(), len(block_sizes), p, M, c.data_ptr(), _lib.BF16, 0, ops._stream(A))
    return c


_LIB.impl("hip_grouped_gemm_single", hip_grouped_gemm_single, "CUDA")
