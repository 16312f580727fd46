"""Single-rank group: the identity collectives of GroupCommunicator at group size 1
(easyinfra/generation/parallel/communicator.py:143-148, 168-172, 270-271), for
running the expert path on one GPU without torch.distributed."""
from __future__ import annotations


class SingleRankGroup:
    group_size = 1
    local_rank = 0
    in_participant = True

    def all_reduce(self, t, *a, **k):
        return t

    def all_gather_into_tensor(self, out, t, *a, **k):
        out.view(-1)[: t.numel()].copy_(t.reshape(-1))
        return out

    def all_to_all_single(self, out, t, *a, **k):
        out.copy_(t)
        return out
