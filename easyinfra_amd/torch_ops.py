"""torch.ops registration of the grouped GEMM for the reference's native op point.

EasyInfra loads ``*.so`` op libraries and calls
``torch.ops.ops.<impl>_grouped_gemm_single(A, B_list, block_sizes)``
(easyinfra/__init__.py:7-20, single_group_gemm_moe.py:53-91): ``A[M,K]`` rows in
contiguous blocks, ``B_list`` one ``[N,K]`` nn.Linear weight per block,
``out[rows_i] = A[rows_i] @ B_i^T``.  Importing this module registers
``torch.ops.ops.hip_grouped_gemm_single`` with that schema, backed by the HIP
grouped GEMM (the weights are stacked into ``[n_blocks, N, K]`` per call unless the
list already consists of consecutive views of one stacked tensor).
"""
from __future__ import annotations

from typing import List

import torch

from . import ops

_LIB = torch.library.Library("ops", "FRAGMENT")
_LIB.define("hip_grouped_gemm_single(Tensor A, Tensor[] B_list, int[] block_sizes) -> Tensor")


def _stack_weights(b_list: List[torch.Tensor]) -> torch.Tensor:
    b0 = b_list[0]
    N, K = b0.shape
    base = b0.untyped_storage().data_ptr()
    contiguous_views = all(b.is_contiguous() and b.shape == b0.shape and b.dtype == b0.dtype and
                           b.untyped_storage().data_ptr() == base and
                           b.data_ptr() == b0.data_ptr() + i * N * K * b0.element_size()
                           for i, b in enumerate(b_list))
    if contiguous_views:
        return torch.as_strided(b0, (len(b_list), N, K), (N * K, K, 1))
    return torch.stack([b.contiguous() for b in b_list], 0)


def hip_grouped_gemm_single(A: torch.Tensor, B_list: List[torch.Tensor], block_sizes: List[int]) -> torch.Tensor:
    if len(B_list) != len(block_sizes):
        raise ValueError(f"{len(B_list)} weights for {len(block_sizes)} blocks")
    M = int(sum(block_sizes))
    if M != A.shape[0]:
        raise ValueError(f"block sizes sum to {M}, A has {A.shape[0]} rows")
    b = _stack_weights(B_list)
    off = torch.zeros(len(block_sizes) + 1, dtype=torch.int32)
    off[1:] = torch.cumsum(torch.tensor(block_sizes, dtype=torch.int64), 0).to(torch.int32)
    return ops.grouped_gemm(A.contiguous(), b, off.to(A.device), M, out_dtype=A.dtype)


_LIB.impl("hip_grouped_gemm_single", hip_grouped_gemm_single, "CUDA")
