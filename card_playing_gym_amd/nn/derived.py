"""Device-side weight copies derived from module parameters, kept current across updates.

The bf16 handles (``cg_trunk``, ``cg_heads``, ``cg_piquet``) hold bf16 copies of fp32
parameters in the kernels' fragment order.  A captured HIP graph replays reading those
copies, so they must follow every in-place change of the parameters, as the reference's
graphs follow them by deriving autocast's casts inside the graph
(cardgym/rl/graphs.py:17-22): the decode graphs of cardgym.rl.continuous persist across
``trainer.update`` (an optimiser step on the same actor) and across ``load_state_dict``
(rl/loop.py:225, rl/async_rollout.py:95).

Three points re-derive the copies of every live handle whose parameters changed (their
version counters moved), on the current stream of the handle's device:

* any optimiser's ``step()`` (a global post-step hook, registered once), for every handle
  over one of that optimiser's parameters whatever the version counters say (fused
  optimisers update in place without moving them);
* ``load_state_dict`` on a module that owns a handle (a post-load hook);
* every eager call that uses the handle, and ``refresh_native()`` on demand (after an
  in-place edit outside an optimiser, e.g. ``with torch.no_grad(): p.mul_(0.5)``).

A handle whose parameters moved (``module.to(other_device)``, ``.double()``, a replaced
Parameter) is retired, not destroyed: a graph captured earlier may still replay against it,
and freeing its device memory would turn that replay into a memory fault.  The native
handles also hold raw pointers into the fp32 parameters themselves (LayerNorm gains and
biases the kernels read directly, the sources of every refresh), and ``Module._apply``
swaps ``param.data`` onto new storage inside the same Parameter objects, so each handle
keeps a detached view of every parameter as it was built: the storage its pointers name
stays allocated until the handle is released with its module.  A handle whose parameters
no longer live where its pointers point is never refreshed again: its copies keep the
weights of the moment the parameters moved.
"""

from __future__ import annotations

import ctypes
import weakref
from typing import Callable, Iterable

import torch
from torch.optim.optimizer import register_optimizer_step_post_hook

_LIVE: "weakref.WeakSet[DerivedCopies]" = weakref.WeakSet()
_HOOKED = False


class DerivedCopies:
    """Base of the bf16 handles: tracks the parameters' storage and version counters."""

    def __init__(self, params: Iterable[torch.Tensor], device: torch.device) -> None:
        self.handle = ctypes.c_void_p()
        self.params = list(params)
        self.device = device
        self.signature = tuple(p.data_ptr() for p in self.params)
        # Detached views share the parameters' current storage and keep it alive after
        # param.data is swapped onto new storage (the native handle points into it).
        self._storage = [p.detach() for p in self.params]
        self.versions = tuple(p._version for p in self.params)
        _LIVE.add(self)
        _install_optimizer_hook()

    # -- subclass interface ------------------------------------------------------

    def _refresh(self, stream: int) -> None:  # pragma: no cover - abstract
        raise NotImplementedError

    def close(self) -> None:  # pragma: no cover - abstract
        raise NotImplementedError

    def current_stream(self) -> int:
        """The device's current stream (where a refresh outside any call is enqueued)."""

        from .kv_cache import stream_handle

        return stream_handle(self.device)

    # -- shared logic ------------------------------------------------------------

    def matches(self, params: list[torch.Tensor]) -> bool:
        """Whether ``params`` are still the tensors (and storage) the copies derive from."""

        return (
            len(params) == len(self.params)
            and tuple(p.data_ptr() for p in params) == self.signature
            and all(a is b for a, b in zip(params, self.params))
        )

    def moved(self) -> bool:
        """Whether any parameter's data now lives elsewhere than the handle's pointers name."""

        return tuple(p.data_ptr() for p in self.params) != self.signature

    def refresh_now(self, stream: int | None = None) -> bool:
        if self.moved():
            return False
        self._refresh(self.current_stream() if stream is None else stream)
        self.versions = tuple(p._version for p in self.params)
        return True

    def refresh_if_changed(self, stream: int | None = None) -> bool:
        versions = tuple(p._version for p in self.params)
        if versions == self.versions or self.moved():
            return False
        self._refresh(self.current_stream() if stream is None else stream)
        self.versions = versions
        return True

    def __del__(self) -> None:  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass


def refresh_all() -> int:
    """Re-derives the copies of every live handle whose parameters changed; returns how many."""

    count = 0
    for handle in list(_LIVE):
        if getattr(handle, "handle", None) and handle.refresh_if_changed():
            count += 1
    return count


def _after_optimizer_step(optimizer, args, kwargs) -> None:
    # Fused optimisers (torch.optim.Adam(fused=True), the reference trainer's choice on CUDA,
    # cardgym/rl/trainer.py:392-395) update parameters without moving their version counters,
    # so every handle over a parameter this optimiser owns is re-derived unconditionally.
    owned = {id(p) for group in optimizer.param_groups for p in group["params"]}
    for handle in list(_LIVE):
        if getattr(handle, "handle", None) and any(id(p) in owned for p in handle.params):
            handle.refresh_now()
    refresh_all()


def _install_optimizer_hook() -> None:
    global _HOOKED
    if not _HOOKED:
        register_optimizer_step_post_hook(_after_optimizer_step)
        _HOOKED = True


def after_load_hook(module, incompatible_keys) -> None:
    """``register_load_state_dict_post_hook`` target: re-derive after new weights land."""

    refresh_all()


class HandleCache:
    """Per-(device, key) handles of one module, with retirement instead of destruction."""

    def __init__(self) -> None:
        self.entries: dict = {}
        self.retired: list[DerivedCopies] = []

    def __reduce__(self):
        # A copied or pickled module starts with no handles: two owners of one raw handle
        # would both destroy it.
        return (HandleCache, ())

    def get(self, key, params: list[torch.Tensor], build: Callable[[], DerivedCopies], stream: int) -> DerivedCopies:
        entry = self.entries.get(key)
        if entry is not None and entry.matches(params):
            entry.refresh_if_changed(stream)
            return entry
        if entry is not None:
            self.retired.append(entry)
        entry = build()
        self.entries[key] = entry
        return entry

    def refresh(self) -> int:
        count = 0
        for entry in [*self.entries.values(), *self.retired]:
            if entry.handle and entry.refresh_if_changed():
                count += 1
        return count

    def retire_moved(self, current: Callable[[object], list[torch.Tensor]]) -> None:
        """After ``Module._apply``: keep handles whose parameters did not move."""

        for key in list(self.entries):
            entry = self.entries[key]
            if not entry.matches(current(key)):
                self.retired.append(self.entries.pop(key))

    def close(self) -> None:
        for entry in [*self.entries.values(), *self.retired]:
            entry.close()
        self.entries, self.retired = {}, []
