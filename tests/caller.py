"""A stand-in for the reference's rollout caller, for the tests only.

The reference's collectors drive an actor through ``cardgym.rl.graphs.DecodeGraphs``
(cardgym/rl/graphs.py:63-151, with cardgym/nn/compile.py:26-44): the wave body -- the
ragged trunk step, then every policy head and the seat values at each row's readout -- is
compiled with ``torch.compile(dynamic=True)``, run once on a side stream, captured into a
CUDA graph and replayed with new inputs copied into the captured input tensors.  The tests
drive this package's model the same way through the helpers here, to show that such a
caller runs the HIP path unchanged: the body compiles as one graph over the ``cardgym_hip``
custom ops (``fullgraph=True``), the capture records the kernels, and replays follow the
pool and the weights.
"""

from __future__ import annotations

from contextlib import nullcontext

import numpy as np
import torch


def wave_body(model, cache, dtype: torch.dtype | None, values: bool = True):
    """The wave as the actor interface computes it (cardgym/games/base.py:25-58), under
    autocast ``dtype`` (None: fp32): fp32 [rows, logits of every head (+ seat values)]."""

    heads = tuple(model.policy_heads)

    def body(tokens, positions, offsets, cache_rows, span: int):
        mixed = nullcontext() if dtype is None else torch.autocast("cuda", dtype=dtype, cache_enabled=False)
        with mixed:
            hidden = model.forward_ragged(tokens, positions, cache, offsets, span=span, rows=cache_rows)
            context = model.pop_context()
            if context is not None:
                context = context[torch.arange(hidden.shape[0], device=hidden.device), offsets]
            parts = [model.policy_logits(hidden, head, None, None, context) for head in heads]
            if values:
                parts.append(model.player_values(hidden))
        return torch.cat([p.float() for p in parts], dim=-1)

    return body


def compiled(body):
    """``torch.compile(dynamic=True, fullgraph=True)``: any graph break fails the compile."""

    return torch.compile(body, dynamic=True, fullgraph=True)


class CapturedWave:
    """One wave shape captured the way the reference's rollout graphs capture it: a warm-up
    call on a side stream, a capture into a CUDA graph over static device inputs, replays
    after the inputs are overwritten in place.  The warm-up appends the wave's K / V once
    and the first replay appends the same K / V again (same rows, positions and values)."""

    def __init__(self, fn, tokens, positions, offsets, cache_rows, span: int) -> None:
        self.inputs = [t.clone() for t in (tokens, positions, offsets, cache_rows)]
        self.span = int(span)
        self.fn = fn
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn(*self.inputs, self.span)
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.output = fn(*self.inputs, self.span)

    def replay(self, tokens, positions, offsets, cache_rows) -> torch.Tensor:
        for static, new in zip(self.inputs, (tokens, positions, offsets, cache_rows)):
            static.copy_(new, non_blocking=True)
        self.graph.replay()
        return self.output


def random_wave(rng: np.random.Generator, capacity: int, rows: int, run: int, max_pos: int, vocab: int = 512):
    """Host arrays of one wave over distinct cache rows: tokens [rows, run, 1], positions,
    readout offsets, cache rows (int64)."""

    cache_rows = rng.permutation(capacity)[:rows]
    positions = rng.integers(0, max_pos, size=rows)
    tokens = rng.integers(0, vocab, size=(rows, run, 1))
    offsets = rng.integers(0, run, size=rows)
    return tokens, positions, offsets, cache_rows


def to_device(device, *arrays):
    return [torch.from_numpy(np.asarray(a, dtype=np.int64)).to(device) for a in arrays]
