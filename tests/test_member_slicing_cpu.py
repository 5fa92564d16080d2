"""Member bookkeeping of Eggroll.population (eggroll.py:133-146) across ranks, on the CPU.

member_plan is what Eggroll.population walks: for every rank of a world the chunks of its members, each chunk's
first direction and its sequence. Checked against the reference's formulas written out member by member
(direction (g mod 2P) // 2, sign + for even g, sequence of the chunk's first member g0 // per_seq, rank r owning
[r per_rank, (r + 1) per_rank)), and through torch.distributed on two gloo ranks: each rank evaluates a stand-in
loss of its members (a function of direction, sign and sequence), the ranks all-gather as eggroll.py:147-150
does, and the gathered vector equals the one-rank evaluation of the whole population."""
import os

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from noise_amd.eggroll import member_plan


def stand_in(plan, pairs):
    """A loss per member that depends on exactly what the member's evaluation depends on."""
    out = []
    for start, n, d0, seq in plan:
        g = torch.arange(start, start + n)
        d = (g % (2 * pairs)) // 2
        assert d[0].item() == d0
        sign = 1 - 2 * (g % 2)
        out.append(d * 1000.0 + sign * 0.5 + seq * 0.001)
    return torch.cat(out)


def reference_losses(pairs, sequences, chunk, world):
    """eggroll.py:133-146 written out per member: rank r's chunks start at r per_rank, every `chunk` members,
    and take the sequence of their first member."""
    members = max(2 * pairs, 2 * sequences)
    per_seq, per_rank = members // sequences, members // world
    g = torch.arange(members)
    d = (g % (2 * pairs)) // 2
    sign = 1 - 2 * (g % 2)
    rank_start = g // per_rank * per_rank
    chunk_start = rank_start + (g - rank_start) // chunk * chunk
    seq = chunk_start // per_seq
    return d * 1000.0 + sign * 0.5 + seq * 0.001


@pytest.mark.parametrize('pairs,sequences,world,chunk', [
    (512, 8, 1, 512), (512, 8, 2, 512), (512, 8, 4, 128), (131072, 8, 2, 512), (4, 8, 2, 2), (6, 3, 2, 4)])
def test_member_plan_matches_reference_formulas(pairs, sequences, world, chunk):
    members = max(2 * pairs, 2 * sequences)
    per_rank = members // world
    got = []
    for rank in range(world):
        plan = member_plan(pairs, sequences, rank, world, chunk)
        assert plan[0][0] == rank * per_rank and sum(c[1] for c in plan) == per_rank
        got.append(stand_in(plan, pairs))
    assert torch.equal(torch.cat(got), reference_losses(pairs, sequences, chunk, world))


def test_member_plan_rejects_odd_chunks():
    with pytest.raises(ValueError):
        member_plan(512, 8, 0, 1, 3)


def _rank_main(rank, world, port, pairs, sequences, chunk, out):
    os.environ.update(MASTER_ADDR='127.0.0.1', MASTER_PORT=str(port))
    dist.init_process_group('gloo', rank=rank, world_size=world)
    try:
        losses = stand_in(member_plan(pairs, sequences, rank, world, chunk), pairs)
        gathered = [torch.empty_like(losses) for _ in range(world)]
        dist.all_gather(gathered, losses)
        if rank == 0:
            torch.save(torch.cat(gathered), out)
    finally:
        dist.destroy_process_group()


def test_two_gloo_ranks_gather_the_population(tmp_path):
    import socket
    with socket.socket() as s:
        s.bind(('127.0.0.1', 0))
        port = s.getsockname()[1]
    pairs, sequences, chunk = 512, 8, 128
    out = str(tmp_path / 'gathered.pt')
    mp.spawn(_rank_main, args=(2, port, pairs, sequences, chunk, out), nprocs=2, join=True)
    gathered = torch.load(out, weights_only=True)
    whole = stand_in(member_plan(pairs, sequences, 0, 1, chunk), pairs)
    assert torch.equal(gathered, whole)  # chunks of 128 never straddle a sequence of 128 members
    assert torch.equal(gathered, reference_losses(pairs, sequences, chunk, 2))
