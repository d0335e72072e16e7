"""The graph-plan cache the drop-in modules use when called without plan=
(maloq_amd.message.plan_for): one plan per edge_index tensor, rebuilt when the
tensor changes.  MessagePlan is host logic (sorts and CSR pointers), so this
runs on CPU tensors."""
import torch

from maloq_amd import message as M


def _graph(seed, E=40, N=9):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, N, (2, E), generator=g), N


def test_same_tensor_same_plan():
    M.clear_plan_cache()
    ei, N = _graph(0)
    built = M._PLANS.built
    p1 = M.plan_for(ei, N)
    for _ in range(4):  # the backbone's layers: one tensor, one plan
        assert M.plan_for(ei, N) is p1
    assert M._PLANS.built == built + 1
    ref = M.MessagePlan(ei, N)
    assert torch.equal(p1.perm, ref.perm) and torch.equal(p1.seg_ptr, ref.seg_ptr)


def test_changed_or_other_tensor_rebuilds():
    M.clear_plan_cache()
    ei, N = _graph(1)
    p1 = M.plan_for(ei, N)
    assert M.plan_for(ei.clone(), N) is not p1          # another tensor, even with equal values
    assert M.plan_for(ei, N + 1) is not p1              # another node count
    ei[1, 0] = (ei[1, 0] + 1) % N                       # in place: the version counter moves
    p2 = M.plan_for(ei, N)
    assert p2 is not p1
    assert torch.equal(p2.perm, M.MessagePlan(ei, N).perm)


def test_cache_is_bounded():
    M.clear_plan_cache()
    graphs = [_graph(s) for s in range(M._PLANS.size + 3)]
    plans = [M.plan_for(ei, N) for ei, N in graphs]
    assert len(M._PLANS._entries) == M._PLANS.size
    ei, N = graphs[-1]
    assert M.plan_for(ei, N) is plans[-1]               # the most recent ones stay
