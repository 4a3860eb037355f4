"""HIP graphs of a rollout decode wave (API of cardgym.rl.graphs).

``DecodeGraphs(model, cache, precision=..., values=...)`` and ``graphs_enabled`` keep the
interface of cardgym/rl/graphs.py:48-151: ``run(tokens, positions, offsets, cache_rows,
span)`` decodes one wave -- a ragged step of every row through the trunk, then every
policy head (and, with ``values``, the seat values) at each row's readout -- and returns
the device output [rows, columns] (fp32; ``columns`` maps each head to its slice).  One
graph per wave shape ``(rows, tokens per row, token width, span)``: the first wave of a
shape compiles the body (``torch.compile(dynamic=True)``, card_playing_gym_amd/nn/compile.py),
runs it once on a side stream with the real inputs, captures it, and replays it; later
waves of the shape copy their inputs into the graph's input buffer and replay.

On this path the body is the custom ops of card_playing_gym_amd/nn/ops.py -- the embedder,
``trunk_step`` (every layer's K / V append, attention and projections), the heads -- plus
the output concatenation, so a replay is one hipGraph launch of those kernels.  The KV
pool and the weights stay where the graph captured them: the cache is fixed for the
collector's layout, and the bf16 weight copies the kernels read are re-derived in place
after optimiser steps and ``load_state_dict`` (card_playing_gym_amd/nn/derived.py).

Graphs share one memory pool and run one at a time on the current stream; a wave's output
must be copied out before the next replay of that shape overwrites it.
"""

from __future__ import annotations

import os
from contextlib import nullcontext
from dataclasses import dataclass

import numpy as np
import torch

from ..nn.compile import compiled

PRECISIONS = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def graphs_enabled(model, device: torch.device) -> bool:
    """A GPU device, a model whose heads read only the readout state, and not switched
    off by CARDGYM_CUDA_GRAPHS=0 (graphs.py:48-56)."""

    return (
        device.type == "cuda"
        and bool(getattr(model, "graphable_heads", False))
        and os.environ.get("CARDGYM_CUDA_GRAPHS", "1") != "0"
    )


@dataclass
class _Captured:
    graph: torch.cuda.CUDAGraph
    inputs: torch.Tensor  # int64 device buffer: tokens, then positions, offsets, cache rows
    output: torch.Tensor  # fp32 [rows, columns]


class DecodeGraphs:
    def __init__(self, model, cache, *, precision: str, values: bool) -> None:
        if precision not in PRECISIONS:
            raise ValueError(f"precision must be one of {sorted(PRECISIONS)}")
        self.model = model
        self.cache = cache
        self.precision = precision
        self.values = values
        self.heads: tuple[str, ...] = tuple(model.policy_heads)
        self.pool = torch.cuda.graph_pool_handle()
        self._forward = compiled(self._outputs, cache.device)
        self._graphs: dict[tuple[int, int, int, int], _Captured] = {}
        self.columns: dict[str, slice] = {}

    def __len__(self) -> int:
        return len(self._graphs)

    def _precision(self):
        if self.precision == "fp32":
            return nullcontext()
        # No cast cache: weight casts derived inside a graph must follow later updates.
        return torch.autocast("cuda", dtype=PRECISIONS[self.precision], cache_enabled=False)

    def _outputs(self, inputs: torch.Tensor, rows: int, run: int, width: int, span: int) -> list[torch.Tensor]:
        """Every head's logits, then the values, at each row's readout (fp32)."""

        cells = rows * run * width
        tokens = inputs[:cells].view(rows, run, width)
        positions, offsets, cache_rows = inputs[cells:].view(3, rows)
        with self._precision():
            hidden = self.model.forward_ragged(tokens, positions, self.cache, offsets, span=span, rows=cache_rows)
            context = self.model.pop_context()
            if context is not None:
                context = context[torch.arange(rows, device=inputs.device), offsets]
            out = [self.model.policy_logits(hidden, head, None, None, context) for head in self.heads]
            if self.values:
                out.append(self.model.player_values(hidden))
        return [o.float() for o in out]

    def _body(self, inputs: torch.Tensor, rows: int, run: int, width: int, span: int) -> torch.Tensor:
        out = self._forward(inputs, rows, run, width, span)
        if not self.columns:
            names = [*self.heads, "values"] if self.values else list(self.heads)
            start = 0
            for name, o in zip(names, out):
                self.columns[name] = slice(start, start + o.shape[-1])
                start += o.shape[-1]
        return torch.cat(out, dim=-1)

    def run(
        self,
        tokens: np.ndarray,
        positions: np.ndarray,
        offsets: np.ndarray,
        cache_rows: np.ndarray,
        span: int,
    ) -> torch.Tensor:
        """Decode one wave of tokens [rows, run, width]; returns the device output
        [rows, columns] (copy it out before the next run of this shape)."""

        rows, run, width = tokens.shape
        span = min(int(span), self.cache.max_len)
        key = (rows, run, width, span)
        packed = np.concatenate(
            [np.asarray(a, dtype=np.int64).reshape(-1) for a in (tokens, positions, offsets, cache_rows)]
        )
        host = torch.from_numpy(packed).pin_memory()
        entry = self._graphs.get(key)
        if entry is None:
            return self._capture(key, host)
        entry.inputs.copy_(host, non_blocking=True)
        entry.graph.replay()
        return entry.output

    def _capture(self, key: tuple[int, int, int, int], host: torch.Tensor) -> torch.Tensor:
        rows, run, width, span = key
        inputs = torch.empty(host.shape, dtype=torch.int64, device=self.cache.device)
        inputs.copy_(host, non_blocking=True)
        # Warm-up on a side stream: compiles the shape if it is new and appends the same
        # K / V the replay appends again (same rows, same positions).
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._body(inputs, rows, run, width, span)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool):
            output = self._body(inputs, rows, run, width, span)
        self._graphs[key] = _Captured(graph, inputs, output)
        graph.replay()
        return output
