"""The refresh machinery of the bf16 weight copies (card_playing_gym_amd/nn/derived.py), on
the CPU with a stand-in handle: which events re-derive the copies, retirement instead of
destruction, and copies of modules that never share a raw handle."""

from __future__ import annotations

import copy
import pickle

import torch
from torch import nn

from card_playing_gym_amd.nn import derived


class FakeCopies(derived.DerivedCopies):
    def __init__(self, params, log):
        super().__init__(params, torch.device("cpu"))
        self.handle = object()
        self.log = log

    def current_stream(self):
        return 0

    def _refresh(self, stream):
        self.log.append(("refresh", id(self)))

    def close(self):
        if self.handle is not None:
            self.log.append(("close", id(self)))
            self.handle = None


class Owner(nn.Module):
    def __init__(self, log):
        super().__init__()
        self.lin = nn.Linear(4, 3)
        self._handles = derived.HandleCache()
        self.register_load_state_dict_post_hook(derived.after_load_hook)
        self.log = log

    def native(self):
        params = [self.lin.weight, self.lin.bias]
        return self._handles.get("cpu", params, lambda: FakeCopies(params, self.log), stream=0)

    def _apply(self, fn, *args, **kwargs):
        out = super()._apply(fn, *args, **kwargs)
        self._handles.retire_moved(lambda key: [self.lin.weight, self.lin.bias])
        return out


def refreshes(log):
    return sum(1 for event in log if event[0] == "refresh")


def test_optimizer_step_and_load_state_dict_refresh_the_copies():
    log = []
    owner = Owner(log)
    handle = owner.native()
    assert owner.native() is handle and refreshes(log) == 0
    owner.lin.weight.grad = torch.ones_like(owner.lin.weight)
    torch.optim.SGD([owner.lin.weight], lr=0.1).step()
    assert refreshes(log) == 1  # the global post-step hook
    # Fused Adam leaves the version counters where they were: the hook refreshes anyway.
    owner.lin.weight.grad = torch.ones_like(owner.lin.weight)
    versions = owner.lin.weight._version
    torch.optim.Adam([owner.lin.weight], lr=0.1, fused=True).step()
    assert owner.lin.weight._version == versions and refreshes(log) == 2
    # An optimiser over other parameters leaves the copies alone.
    other = torch.nn.Parameter(torch.zeros(2))
    other.grad = torch.ones(2)
    torch.optim.Adam([other], lr=0.1, fused=True).step()
    assert refreshes(log) == 2
    owner.load_state_dict({k: v + 1 for k, v in owner.state_dict().items()})
    assert refreshes(log) == 3  # the post-load hook
    owner.native()
    assert refreshes(log) == 3  # nothing changed since
    with torch.no_grad():
        owner.lin.bias.mul_(2)
    owner.native()  # an eager call notices the version counter
    assert refreshes(log) == 4
    with torch.no_grad():
        owner.lin.bias.mul_(2)
    assert owner._handles.refresh() == 1 and refreshes(log) == 5


def test_moved_parameters_retire_the_handle_without_destroying_it():
    log = []
    owner = Owner(log)
    first = owner.native()
    owner.to(torch.device("cpu"))  # nothing moves: the handle stays
    assert owner.native() is first
    owner.double()  # parameters replaced: retired, a new handle for new calls
    second = owner.native()
    assert second is not first and first in owner._handles.retired
    assert not [e for e in log if e[0] == "close"]
    # The storage `first` points into outlives the swap of param.data: a graph captured
    # before the move still reads it.
    assert [t.data_ptr() for t in first._storage] == list(first.signature)
    assert first.moved() and not second.moved()
    # The moved parameters are no longer what `first` points into: updates to them never
    # refresh it (no eager call, no optimiser step, no refresh_all).
    before = refreshes(log)
    with torch.no_grad():
        first.params[0].add_(1)
    derived.refresh_all()
    first.params[0].grad = torch.ones_like(first.params[0])
    torch.optim.SGD([first.params[0]], lr=0.1).step()
    assert ("refresh", id(first)) not in log
    assert not first.refresh_now() and not first.refresh_if_changed()
    # `second` owns the moved parameters: refresh_all after the in-place edit, then the step.
    assert log[-2:] == [("refresh", id(second))] * 2 and refreshes(log) == before + 2
    owner._handles.close()
    assert {("close", id(first)), ("close", id(second))} <= set(log)


def test_copies_of_a_module_start_without_handles():
    log = []
    owner = Owner(log)
    owner.native()
    clone = copy.deepcopy(owner)
    assert clone._handles.entries == {} and clone._handles.retired == []
    restored = pickle.loads(pickle.dumps(owner._handles))
    assert restored.entries == {}
