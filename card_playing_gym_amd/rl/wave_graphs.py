"""Per-shape HIP graphs of a rollout decode wave.

A rollout collector decodes waves of a few recurring shapes: ``rows`` cache rows, each
appending ``run`` tokens of ``width`` ids, read back through a ``span`` bucket.  Every
launch of such a wave on this path is a native call behind a torch custom op (embedding,
the whole trunk step, the heads), so a wave needs no compiler to become one replayable
graph: ``WaveGraphs`` records the launches themselves, one HIP graph per shape, and
replays it for every later wave of that shape.  The constructor and ``run`` take what the
rollout graphs of ``cardgym.rl.graphs.DecodeGraphs`` take (cardgym/rl/graphs.py:63-131:
``(model, cache, precision=, values=)``, ``run(tokens, positions, offsets, cache_rows,
span)`` returning the device rows of every head's logits, then the seat values, with
``columns`` naming each head's slice), so a collector can hold either.

How a shape is taken on:

* Its first wave runs **eagerly**.  That creates whatever the launches need and may not
  be created under capture (the bf16 weight handles, which allocate device memory) and
  gives the wave's output.  The same launches are then **captured without running** (a
  capture records; it does not execute), so the wave's K / V append happens once, not
  twice.
* Later waves write their host arrays straight into the shape's **pinned staging buffer**
  (allocated once per shape, not per wave), issue one host-to-device copy and one graph
  launch on the current stream.  The staging buffer is rewritten only after the event
  recorded behind the previous copy out of it has completed.
* At most ``max_graphs`` shapes are held; taking on one more releases the least recently
  used (its graph, its buffers).

Weights: the graph reads the bf16 copies the model's handles keep, which follow optimiser
steps and ``load_state_dict`` in place (card_playing_gym_amd/nn/derived.py), so a replay
after a weight update uses the new weights.  The KV pool is the one given at construction.
A replay overwrites the shape's output buffer: copy it out before the next wave of that
shape.  Graphs run one at a time, on the stream current at ``run``.
"""

from __future__ import annotations

from collections import OrderedDict
from contextlib import nullcontext
from dataclasses import dataclass

import numpy as np
import torch

AUTOCAST = {"bf16": torch.bfloat16, "fp16": torch.float16}


@dataclass
class _Shape:
    graph: torch.cuda.CUDAGraph
    staging: torch.Tensor  # pinned int64 host buffer: tokens, positions, offsets, cache rows
    host: np.ndarray  # numpy view of ``staging``
    inputs: torch.Tensor  # its device twin, read by the graph
    output: torch.Tensor  # fp32 [rows, columns], written by every replay
    copied: torch.cuda.Event  # recorded behind the last copy out of ``staging``


class WaveGraphs:
    """One captured HIP graph per decode-wave shape (see the module docstring)."""

    def __init__(self, model, cache, *, precision: str, values: bool, max_graphs: int = 64) -> None:
        if precision != "fp32" and precision not in AUTOCAST:
            raise ValueError(f"precision must be 'fp32', 'bf16' or 'fp16', not {precision!r}")
        if max_graphs < 1:
            raise ValueError("max_graphs must be at least 1")
        self.model = model
        self.cache = cache
        self.precision = precision
        self.values = bool(values)
        self.max_graphs = int(max_graphs)
        self.pool = torch.cuda.graph_pool_handle()
        self.columns: dict[str, slice] = {}
        self._shapes: "OrderedDict[tuple[int, int, int, int], _Shape]" = OrderedDict()

    def __len__(self) -> int:
        return len(self._shapes)

    def clear(self) -> None:
        """Releases every captured shape (e.g. before the pool or the model is replaced)."""

        torch.cuda.current_stream(self.cache.device).synchronize()
        self._shapes.clear()

    # -- the wave ----------------------------------------------------------------------

    def _mixed(self):
        if self.precision == "fp32":
            return nullcontext()
        # No cast cache: a cast made inside a captured graph would be replayed stale.
        return torch.autocast("cuda", dtype=AUTOCAST[self.precision], cache_enabled=False)

    def _wave(self, inputs: torch.Tensor, key: tuple[int, int, int, int]) -> torch.Tensor:
        """Trunk step and heads of one wave from the packed device inputs -> fp32 [rows, columns]."""

        rows, run, width, span = key
        n = rows * run * width
        tokens = inputs[:n].view(rows, run, width)
        positions, offsets, cache_rows = inputs[n : n + rows], inputs[n + rows : n + 2 * rows], inputs[n + 2 * rows :]
        model = self.model
        with self._mixed():
            hidden = model.forward_ragged(tokens, positions, self.cache, offsets, span=span, rows=cache_rows)
            named = self._readout(hidden, offsets)
        if not self.columns:
            start = 0
            for name, part in named:
                self.columns[name] = slice(start, start + part.shape[-1])
                start += part.shape[-1]
        return torch.cat([part.float() for _, part in named], dim=-1)

    def _readout(self, hidden: torch.Tensor, offsets: torch.Tensor) -> list[tuple[str, torch.Tensor]]:
        model = self.model
        heads = tuple(model.policy_heads)
        fused = getattr(model, "readout_heads", None)
        if fused is not None:
            # One launch for every head of the model (the synthetic model's fused heads).
            return list(fused(hidden, heads, self.values).items())
        context = model.pop_context()
        if context is not None:
            context = context[torch.arange(hidden.shape[0], device=hidden.device), offsets]
        named = [(head, model.policy_logits(hidden, head, None, None, context)) for head in heads]
        if self.values:
            named.append(("values", model.player_values(hidden)))
        return named

    # -- shapes ------------------------------------------------------------------------

    def run(self, tokens, positions, offsets, cache_rows, span: int) -> torch.Tensor:
        """Decode one wave of ``tokens`` [rows, run, width] (host arrays); returns the device
        output [rows, columns], valid until the next wave of the same shape."""

        tokens = np.asarray(tokens)
        rows, run, width = tokens.shape
        key = (rows, run, width, min(int(span), self.cache.max_len))
        shape = self._shapes.get(key)
        fresh = shape is None
        if fresh:
            shape = self._stage(key)
        else:
            self._shapes.move_to_end(key)
            shape.copied.synchronize()  # the previous wave's copy out of the staging buffer is done
        host, n = shape.host, tokens.size
        host[:n] = tokens.reshape(-1)
        host[n : n + rows] = np.asarray(positions).reshape(-1)
        host[n + rows : n + 2 * rows] = np.asarray(offsets).reshape(-1)
        host[n + 2 * rows :] = np.asarray(cache_rows).reshape(-1)
        stream = torch.cuda.current_stream(self.cache.device)
        shape.inputs.copy_(shape.staging, non_blocking=True)
        shape.copied.record(stream)
        if not fresh:
            shape.graph.replay()
            return shape.output
        out = self._wave(shape.inputs, key)  # eager: creates handles, appends, gives the output
        self._capture(key, shape)
        return out

    def _stage(self, key: tuple[int, int, int, int]) -> _Shape:
        rows, run, width, _ = key
        size = rows * run * width + 3 * rows
        staging = torch.empty(size, dtype=torch.int64, pin_memory=True)
        inputs = torch.empty(size, dtype=torch.int64, device=self.cache.device)
        return _Shape(None, staging, staging.numpy(), inputs, None, torch.cuda.Event())

    def _capture(self, key: tuple[int, int, int, int], shape: _Shape) -> None:
        while len(self._shapes) >= self.max_graphs:
            self._shapes.popitem(last=False)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool):
            output = self._wave(shape.inputs, key)
        shape.graph, shape.output = graph, output
        self._shapes[key] = shape


# The name the reference's collectors hold their wave graphs under.
DecodeGraphs = WaveGraphs
