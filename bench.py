"""Benchmark: game-tokens/s of the KV-cached ragged trunk step at 4096 games (config 3).

One step = every one of 4096 concurrent games appends one token: embedding + input RMSNorm,
16 decoder blocks (LN + QKV + KV append, ragged GQA decode attention over each game's own
prefix, out-proj + residual, LN + MLP), final LayerNorm at the readouts, then the policy
logits and seat-value heads -- replayed as one HIP graph per step, with the cache, weights
and every step's token ids resident in HBM before the timed region.

Also reported (one JSON line on stdout):
  * roofline: decode attention's algorithmic bytes per launch / its average duration,
    measured live with HIP events on the launch stream, against the 8 TB/s HBM peak;
  * cpu_baseline: the reference path restated in eager PyTorch (oracle/), on the host
    cores, on a bounded sample of the same workload;
  * reference_gpu: the same restatement on the MI355X, eager and captured in a HIP graph;
  * sampling: device policy sampling of the step's logits (masked softmax + inverse CDF);
  * compaction: KVCache.copy_rows as self-play compacts the pool after games end;
  * prefill: forward_prefill throughput at two shapes, beside the reference path on the GPU;
  * piquet_embed: the Piquet token embedder on one 4096-token wave, beside the reference path;
  * piquet_wave: a whole Piquet wave (embedder + 16-layer Piquet trunk step), graph-replayed;
  * train_step: a training step (full causal forward + backward) of the 16-layer trunk, fp32 and bf16 autocast.

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 10]
"""

from __future__ import annotations

import argparse
import json
import os
import signal
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "decode_attention_traffic.json"


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=256)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default="cfg3", choices=["cfg3", "cfg4", "cfg5"])
    p.add_argument("--cpu-games", type=int, default=1024)
    p.add_argument("--cpu-steps", type=int, default=4)
    p.add_argument("--ref-steps", type=int, default=8)
    p.add_argument("--no-baselines", action="store_true")
    p.add_argument("--no-workloads", action="store_true", help="skip the config 4 / 5 lines")
    p.add_argument(
        "--traffic-probe", action="store_true",
        help="run only the decode-attention launches of the timed steps and a 256 MiB calibration copy "
        "(for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes), then exit",
    )
    p.add_argument(
        "--gemm-probe", action="store_true",
        help="time the training step's fp32 GEMM shapes (ours beside torch.matmul, i.e. hipBLASLt) and exit "
        "(for rocprofv3 --pmc passes over the GEMM kernels)",
    )
    p.add_argument(
        "--step-probe", action="store_true",
        help="run only the workload's graph-replayed steps (no baselines, no other rows), print their timing "
        "and exit (for rocprofv3 counter and trace passes over the step's kernels)",
    )
    p.add_argument(
        "--compaction-probe", action="store_true",
        help="run only the KV-compaction measurement on the workload's pool, print it and exit "
        "(for rocprofv3 trace passes over the copy kernels)",
    )
    p.add_argument(
        "--train-probe", action="store_true",
        help="run only the fp32 training step (our path, no reference) and print its timings, then exit "
        "(for a rocprofv3 kernel trace of the training kernels)",
    )
    return p.parse_args()


class Bench:
    """Device-resident state of one workload on cuda:0."""

    def __init__(self, name: str, steps: int, warmup: int) -> None:
        from card_playing_gym_amd.synthetic import WORKLOADS, Driver, build_model

        self.workload = w = WORKLOADS[name]
        self.config = w.trunk_config()
        self.device = torch.device("cuda", 0)
        total = steps + warmup
        self.max_len = w.max_len(total)
        self.model = build_model(self.config, seed=0, device=self.device)
        driver = Driver(w, seed=0, max_len=self.max_len)
        plans = [driver.step() for _ in range(total)]
        self.plans = plans
        dev = self.device
        self.chunks = w.mode == "chunks"
        # Every step's descriptors, resident before timing.  Packed chunks differ in token
        # count from step to step: one tensor per step (and one graph per step).
        if self.chunks:
            self.tokens = [torch.from_numpy(p.tokens).to(dev) for p in plans]
            self.seq_starts = [torch.from_numpy(p.seq_start).to(dev) for p in plans]
            self.readouts = [torch.from_numpy(p.readout).to(dev) for p in plans]
        else:
            self.tokens = torch.from_numpy(np.stack([p.tokens for p in plans])).to(dev)
        self.positions_all = torch.from_numpy(np.stack([p.positions for p in plans])).to(dev)
        self.rows_all = torch.from_numpy(np.stack([p.rows for p in plans])).to(dev)
        games = w.games
        self.games = games
        self.cache = self.model.new_cache(w.capacity(), self.max_len, w.kv_dtype)
        gen = torch.Generator(device=dev).manual_seed(0)
        for k, v in zip(self.cache.k, self.cache.v):
            k.normal_(generator=gen)
            v.normal_(generator=gen)
        self.gathered = w.mode == "continuous"
        # The graph reads a step's inputs from one [parts, games] buffer (tokens, positions
        # and, for gathered rows, the rows) that one copy per step fills.
        self.inputs_all = None
        if self.chunks:
            self.in_buf = torch.zeros((1, games), dtype=torch.int64, device=dev)
            self.tok_buf = torch.zeros((games, 1, 1), dtype=torch.int64, device=dev)
        else:
            parts = [self.tokens.reshape(total, games), self.positions_all]
            if self.gathered:
                parts.append(self.rows_all)
            self.inputs_all = torch.stack(parts, 1).contiguous()
            self.in_buf = torch.zeros((len(parts), games), dtype=torch.int64, device=dev)
            self.tok_buf = self.in_buf[0].view(games, 1, 1)
        self.pos_buf = self.in_buf[1] if not self.chunks else self.in_buf[0]
        self.rows_buf = self.in_buf[2] if self.gathered else torch.arange(games, dtype=torch.int64, device=dev)
        self.readout = torch.zeros(games, dtype=torch.int64, device=dev)
        self.graph = None
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}

    def body(self, step: int = 0):
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=self.workload.precision == "bf16"):
            if self.chunks:
                hidden = self.model.forward_packed(self.tokens[step][:, None], self.seq_starts[step], self.pos_buf,
                                                   self.cache, self.readouts[step])
            else:
                hidden = self.model.forward_ragged(
                    self.tok_buf, self.pos_buf, self.cache, self.readout,
                    rows=self.rows_buf if self.gathered else None,
                )
            return self.model.heads(hidden)

    def load(self, step: int) -> None:
        if self.chunks:
            self.pos_buf.copy_(self.positions_all[step], non_blocking=True)
        else:
            self.in_buf.copy_(self.inputs_all[step], non_blocking=True)

    def capture(self, steps=(0,)) -> None:
        """One graph of the whole step (every step shares it), or for packed chunks one per
        step in `steps` (their token counts differ), sharing one memory pool."""

        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            self.body(steps[0])
        torch.cuda.current_stream().wait_stream(side)
        if not self.chunks:
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph), torch.no_grad():
                self.outputs = self.body()
            return
        pool = torch.cuda.graph_pool_handle()
        for step in steps:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool), torch.no_grad():
                self.outputs = self.body(step)
            self.graphs[step] = graph

    def step(self, step: int) -> None:
        self.load(step)
        (self.graphs[step] if self.chunks else self.graph).replay()

    def tokens_in(self, first: int, count: int) -> int:
        return sum(self.plans[s].n_tokens for s in range(first, first + count))


def traffic_record(workload: str, steps: int, warmup: int, bytes_per_launch: float, kernel: str):
    """HBM bytes per decode-attention launch from the committed counter passes
    (FETCH_SIZE / WRITE_SIZE, calibrated on a plain copy) for this exact run: same workload,
    step count and warm-up, the same kernel and the same algorithmic bytes."""

    if not TRAFFIC_FILE.exists():
        return None
    for record in json.loads(TRAFFIC_FILE.read_text()).get("records", []):
        if (record.get("workload"), record.get("steps"), record.get("warmup"), record.get("kernel")) != (
                workload, steps, warmup, kernel):
            continue
        if abs(record.get("algorithmic_bytes_per_launch", 0) - bytes_per_launch) <= 0.001 * bytes_per_launch:
            return record.get("bytes_per_launch")
    return None


def attention_roofline(bench: Bench, first: int, count: int) -> dict:
    """Average duration and algorithmic bytes of the decode-attention launches of steps
    first..first+count-1, replayed on their own (each step's launches in a HIP graph, as the
    step runs them) between HIP events on the launch stream (packed chunks through the packed
    entry point, as the step launches them)."""

    from card_playing_gym_amd.nn.decode import (
        attention_into, attention_packed_into, attention_packed_order)
    from card_playing_gym_amd.synthetic import kv_bytes

    cfg = bench.config
    dev = bench.device
    games, H, D = bench.games, cfg.n_heads, cfg.head_dim
    tokens = max(p.n_tokens for p in bench.plans[first:first + count])
    # The step's query type: packed chunks store q in the pool's 16-bit type, one-token
    # decode keeps fp32 q (the rule of trunk_forward in csrc/trunk.hip).
    q_dtype = bench.cache.dtype if bench.chunks and bench.cache.dtype != torch.float32 else torch.float32
    q = torch.randn((tokens, H, D), device=dev, dtype=torch.float32).to(q_dtype)
    out = torch.empty((tokens, H, D), device=dev, dtype=torch.bfloat16)
    # Packed chunks: the trunk computes each step's unit order once, before the layers
    # (longest units first): here before the timed launches.  Decode steps run unordered.
    orders = {}
    if bench.chunks:
        for step in range(first, first + count):
            orders[step] = attention_packed_order(
                bench.cache.k[0], bench.rows_all[step], bench.positions_all[step], bench.seq_starts[step],
                bench.plans[step].n_tokens, H, bench.max_len)
    # Each step's launches are captured in a HIP graph of their own (as the step runs them,
    # inside its graph), over that step's own rows and key lengths; the graphs are then
    # replayed back to back between two events on the launch stream.
    stream = torch.cuda.current_stream()
    total_bytes = 0
    itemsize = bench.cache.dtype.itemsize
    graphs, held = [], []
    for i in range(count):
        step = first + i
        plan = bench.plans[step]
        rows_i = bench.rows_all[step].clone()
        if bench.chunks:
            lengths_i = bench.positions_all[step].clone()
            n = plan.n_tokens

            def launches(step=step, n=n, rows_i=rows_i, lengths_i=lengths_i):
                for layer in range(cfg.n_layers):
                    attention_packed_into(out[:n], q[:n], bench.cache.k[layer], bench.cache.v[layer], rows_i,
                                          lengths_i, bench.seq_starts[step], bench.max_len, D ** -0.5, orders[step])
        else:
            lengths_i = bench.positions_all[step] + 1

            def launches(rows_i=rows_i, lengths_i=lengths_i):
                for layer in range(cfg.n_layers):
                    attention_into(out.view(games, H, 1, D), q.view(games, H, 1, D), bench.cache.k[layer],
                                   bench.cache.v[layer], rows_i if bench.gathered else None, lengths_i,
                                   bench.max_len, D ** -0.5)
        if i == 0:
            launches()  # once eagerly, outside any capture
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            launches()
        graphs.append(graph)
        held.append((rows_i, lengths_i))
        kv = kv_bytes(plan, cfg.n_layers, cfg.n_kv_heads, D, itemsize)
        total_bytes += kv + cfg.n_layers * plan.n_tokens * H * D * (q.element_size() + 2)  # + q read + out write (bf16)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for graph in graphs:
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    launches = count * cfg.n_layers
    avg_us = ms * 1e3 / launches
    bytes_per_launch = total_bytes / launches
    achieved = bytes_per_launch / (avg_us * 1e-6) / 1e9
    # Query tiles of 16 per (row, KV head) unit: one for a decode token's 4 heads, four for
    # chunks of up to 16 tokens.
    kernel = "decode_attention_tr_kernel<bf16,32,4>" if bench.chunks else "decode_attention_tr_kernel<bf16,32,1>"
    return {
        "kernel": kernel,
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic_record(bench.workload.name, count, first, bytes_per_launch, kernel),
        "avg_launch_us": round(avg_us, 2),
        "algorithmic_bytes_per_launch": int(bytes_per_launch),
        "launches": launches,
    }


def sampling_time(bench: Bench, reps: int = 20) -> dict:
    """Device policy sampling of the last step's logits (masked softmax + inverse-CDF pick,
    cardgym/rl/ppo.py:75-94) with a random legal mask: HIP events around `reps` calls on
    the current stream."""

    from card_playing_gym_amd.rl import masked_probabilities, sample_rows

    logits = bench.outputs[0]
    rows, width = logits.shape
    gen = torch.Generator(device=bench.device).manual_seed(1)
    mask = torch.rand((rows, width), generator=gen, device=bench.device) < 0.4
    mask[:, 0] = True
    uniforms = torch.rand(rows, generator=gen, device=bench.device, dtype=torch.float64)
    sample_rows(masked_probabilities(logits, mask), mask, uniforms)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        sample_rows(masked_probabilities(logits, mask), mask, uniforms)
    end.record()
    torch.cuda.synchronize()
    # Between events on the stream: includes each call's launch gaps (two ctypes calls and
    # two allocations from Python), so it bounds the kernels' time from above.
    return {"rows": rows, "width": width, "event_us_per_call": round(start.elapsed_time(end) * 1e3 / reps, 2)}


def compaction_time(bench: Bench, reps: int = 5) -> dict:
    """KV compaction as self-play runs it after games end (cardgym/rl/selfplay.py:353-372):
    2048 two-seat games fill the 4096-row pool, 1/64 of them end, and every later game's
    rows slide down over the gap, copying the cache's full prefix length.  Timed with HIP
    events around `reps` calls; indices on the device (the pool classifies the chunk there)
    and on the host (classified before upload)."""

    cache = bench.cache
    seats, games = 2, cache.capacity // 2
    rng = np.random.default_rng(2)
    alive = rng.random(games) >= 1 / 64
    alive[0] = False  # at least one gap, ahead of almost every survivor
    base = np.flatnonzero(alive) * seats
    new = np.arange(base.size) * seats
    moved = base != new
    sources = (base[moved, None] + np.arange(seats)).reshape(-1)
    targets = (new[moved, None] + np.arange(seats)).reshape(-1)
    length = cache.max_len
    moved_bytes = 2 * sources.size * cache.n_layers * 2 * cache.kv_heads * length * cache.head_dim * cache.dtype.itemsize
    out = {"pairs": int(sources.size), "length": length, "layers": cache.n_layers,
           "algorithmic_bytes": moved_bytes}
    for where in ("device", "host"):
        src = torch.from_numpy(sources)
        dst = torch.from_numpy(targets)
        if where == "device":
            src, dst = src.to(bench.device), dst.to(bench.device)
        cache.copy_rows(src, dst, length)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            cache.copy_rows(src, dst, length)
        end.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1e3 / reps
        out[f"{where}_indices_us"] = round(us, 1)
        out[f"{where}_indices_gbs"] = round(moved_bytes / us / 1e3, 1)
    out["frac_of_peak"] = round(out["device_indices_gbs"] / HBM_PEAK_GBS, 4)
    return out


def prefill_time(bench: Bench, with_reference: bool, reps: int = 3) -> dict:
    """Prefill (SequenceModel.forward_prefill, cardgym/nn/trunk.py:376-389) of fresh rows of
    the bench's pool: 4096 games x 16 tokens and 64 games x 512 tokens, bf16, wall time
    over `reps` calls after one untimed call; with `with_reference`, the oracle's restated
    reference path on the same GPU for the same shapes."""

    from oracle.reference_path import RefCache, RefSynthetic, ref_config_of

    cfg, dev = bench.config, bench.device
    out = {}
    ref = rcache = None
    if with_reference:
        state = {k: v.detach() for k, v in bench.model.state_dict().items()}
        ref = RefSynthetic(state, ref_config_of(cfg), "bf16")
        rcache = RefCache(cfg.n_layers, cfg.n_kv_heads, cfg.head_dim, 4096, 512, torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(4)

    def wall(fn) -> float:
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / reps

    for games, length in ((4096, 16), (64, 512)):
        tokens = torch.randint(0, 512, (games, length, 1), generator=gen, device=dev)
        rows = torch.arange(games, device=dev)

        def ours():
            with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
                bench.model.forward_prefill(tokens, bench.cache, rows)

        entry = {"tokens_per_s": round(games * length / wall(ours), 1)}
        if ref is not None:
            def theirs():
                with torch.no_grad():
                    ref.forward_prefill(tokens, rcache, rows)

            entry["reference_gpu_tokens_per_s"] = round(games * length / wall(theirs), 1)
            entry["speedup"] = round(entry["tokens_per_s"] / entry["reference_gpu_tokens_per_s"], 2)
        out[f"{games}x{length}"] = entry
    return out


def piquet_embed_time(device: torch.device, with_reference: bool, tokens: int = 4096, reps: int = 20) -> dict:
    """Piquet's token embedder (cardgym/games/piquet/model.py:286-341: 32 field lookups into
    three tables, the card grid, the summary) for one rollout wave of `tokens` tokens of the
    16-layer actor (d_model 256, PLE 16 x 64, alternating value embeddings, 2 grid blocks),
    HIP events around `reps` calls; with `with_reference`, the oracle's restatement of the
    reference's CUDA path (one-hot GEMM, unfused grid) on the same GPU."""

    from card_playing_gym_amd.games.piquet import PiquetEmbedding, PiquetModelConfig

    config = PiquetModelConfig()
    tc = config.trunk()
    module = PiquetEmbedding(config, tc.ple_width, tc.value_width).to(device)
    g = torch.Generator().manual_seed(5)
    from card_playing_gym_amd.games.piquet import CARD_VOCAB, FIELD_VOCAB, NUM_CARDS

    fields = torch.stack([torch.randint(0, v, (tokens,), generator=g) for v in FIELD_VOCAB], dim=1)
    codes = torch.randint(0, CARD_VOCAB, (tokens, NUM_CARDS), generator=g)
    batch = torch.cat([fields, codes], dim=1).to(device)

    def ours():
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            module(batch)

    def timed(fn) -> float:
        fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) * 1e3 / reps

    us = timed(ours)
    out = {"tokens": tokens, "us_per_wave": round(us, 2), "tokens_per_s": round(tokens / us * 1e6, 1)}
    if with_reference:
        from oracle.piquet import RefPiquetEmbedding

        state = {"embedding." + k: v.detach() for k, v in module.state_dict().items()}
        ref = RefPiquetEmbedding(state, config.card_layers, config.card_kernel, "bf16")

        def theirs():
            with torch.no_grad():
                ref.forward(batch)

        ref_us = timed(theirs)
        out["reference_gpu_us_per_wave"] = round(ref_us, 2)
        out["speedup"] = round(ref_us / us, 2)
    return out


def piquet_wave_time(bench: Bench, with_reference: bool, steps: int = 20) -> dict:
    """A Piquet rollout wave: 4096 games each append one token, embedded by the Piquet
    embedder and run through the 16-layer Piquet trunk (d_ff 512, PLE 64, alternating value
    embeddings; model.py:79-112) with the same context lengths as the bench's middle step,
    the whole wave captured in one HIP graph and replayed `steps` times (wall time).  With
    `with_reference`, the oracle's restated reference path for the same wave, graph-captured."""

    from card_playing_gym_amd.games.piquet import CARD_VOCAB, FIELD_VOCAB, NUM_CARDS, PiquetEmbedding, PiquetModelConfig
    from card_playing_gym_amd.nn.trunk import Trunk

    dev, games = bench.device, bench.games
    config = PiquetModelConfig()
    tc = config.trunk()
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(7)
        emb = PiquetEmbedding(config, tc.ple_width, tc.value_width)
        trunk = Trunk(tc)
    emb, trunk = emb.to(dev).eval(), trunk.to(dev).eval()
    g = torch.Generator().manual_seed(8)
    fields = torch.stack([torch.randint(0, v, (games,), generator=g) for v in FIELD_VOCAB], dim=1)
    codes = torch.randint(0, CARD_VOCAB, (games, NUM_CARDS), generator=g)
    tokens = torch.cat([fields, codes], dim=1).view(games, 1, -1).to(dev)
    middle = len(bench.plans) // 2
    positions = torch.from_numpy(bench.plans[middle].positions).to(dev)
    readout = torch.zeros(games, dtype=torch.int64, device=dev)
    max_len = bench.max_len
    cache = trunk_cache = None
    from card_playing_gym_amd.nn.kv_cache import KVCache

    trunk_cache = KVCache(n_layers=tc.n_layers, kv_heads=tc.n_kv_heads, head_dim=tc.head_dim, capacity=games,
                          max_len=max_len, device=dev, dtype=torch.bfloat16)

    def body():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            x, ple, values = emb(tokens)
            return trunk.forward_ragged(*trunk.condition(x, ple, values), trunk_cache, positions, readout)

    def graphed(fn) -> float:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    with torch.no_grad():
        t = graphed(body)
    out = {"games": games, "ms_per_wave": round(t * 1e3, 4), "game_tokens_per_s": round(games / t, 1),
           "trunk": "16 layers, d 256, 8/2 heads, d_ff 512, PLE 64, alternating VE, bf16 KV"}
    del trunk_cache
    if with_reference:
        from oracle.piquet import RefPiquetEmbedding
        from oracle.reference_path import RefCache, RefTrunk, ref_config_of

        ref_emb = RefPiquetEmbedding({"embedding." + k: v.detach() for k, v in emb.state_dict().items()},
                                     config.card_layers, config.card_kernel, "bf16")
        ref = RefTrunk({"trunk." + k: v.detach() for k, v in trunk.state_dict().items()}, ref_config_of(tc), "bf16")
        cache = RefCache(tc.n_layers, tc.n_kv_heads, tc.head_dim, games, max_len, torch.bfloat16, device=dev)
        span = min(int(-(-(int(bench.plans[middle].positions.max()) + 1) // 32) * 32), max_len)

        def ref_body():
            x, ple, values, _ = ref_emb.forward(tokens)
            return ref.forward_ragged(*ref.condition(x, ple, values), cache, positions, readout, span=span)

        with torch.no_grad():
            rt = graphed(ref_body)
        out["reference_gpu_ms_per_wave"] = round(rt * 1e3, 4)
        out["speedup"] = round(rt / t, 2)
        del cache
    torch.cuda.empty_cache()
    return out


def train_step_time(bench: Bench, with_reference: bool, warmup: int = 3, reps: int = 5) -> dict:
    """One PPO-update-shaped training step of the 16-layer trunk: a full causal forward over a
    batch of sequences, a loss on every hidden state and the backward into every parameter and
    the input (trunk.py:348-374 under autograd), in fp32 (the reference's default precision)
    and under bf16 autocast (its "bf16" precision, cardgym/core/devices.py:32-43).  Wall time
    per step after `warmup` steps; with `with_reference`, the oracle's restatement of the
    reference path (SDPA, autograd; under the same autocast) on the same GPU."""

    from card_playing_gym_amd.nn.trunk import Trunk

    dev, cfg = bench.device, bench.config
    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(11)
        trunk = Trunk(cfg)
    trunk = trunk.to(dev).train()
    ref = None
    if with_reference:
        from oracle.reference_path import RefTrunk, ref_config_of

        state = {"trunk." + k: v.detach().clone().requires_grad_() for k, v in trunk.state_dict().items()}
        ref = RefTrunk(state, ref_config_of(cfg), "fp32")  # autocast applies the bf16 policy itself
    out = {}
    for precision in ("fp32", "bf16"):
        autocast = torch.autocast("cuda", dtype=torch.bfloat16, enabled=precision == "bf16")
        result = {}
        for batch, length in ((256, 64), (64, 256)):
            g = torch.Generator(device=dev).manual_seed(batch)
            x = torch.randn((batch, length, cfg.d_model), generator=g, device=dev).requires_grad_()
            w = torch.randn((batch, length, cfg.d_model), generator=g, device=dev)

            def ours():
                with autocast:
                    h = trunk(*trunk.condition(x, None, None))
                (h * w).sum().backward()

            def theirs():
                with autocast:
                    h = ref.forward_full(*ref.condition(x, None, None))
                (h * w).sum().backward()

            def wall(fn) -> float:
                for _ in range(warmup):
                    fn()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for _ in range(reps):
                    fn()
                torch.cuda.synchronize()
                return (time.perf_counter() - t0) / reps

            entry = {"tokens": batch * length, "ms_per_step": round(wall(ours) * 1e3, 3)}
            entry["tokens_per_s"] = round(batch * length / entry["ms_per_step"] * 1e3, 1)
            if ref is not None:
                entry["reference_gpu_ms_per_step"] = round(wall(theirs) * 1e3, 3)
                entry["speedup"] = round(entry["reference_gpu_ms_per_step"] / entry["ms_per_step"], 2)
            result[f"{batch}x{length}"] = entry
            trunk.zero_grad(set_to_none=True)
        # A ragged microbatch as each trainer runs it (cardgym/rl/trainer.py:652-667): packed rows
        # here (SequenceModel.packs is True on the ROCm GPU), padded to the longest sequence in
        # the reference (its packs() is True only with the MPS Metal trunk).
        lengths = np.random.default_rng(5).integers(32, 257, size=96)
        starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
        n_real, longest = int(lengths.sum()), int(lengths.max())
        g = torch.Generator(device=dev).manual_seed(5)
        xp = torch.randn((n_real, cfg.d_model), generator=g, device=dev).requires_grad_()
        wp = torch.randn((n_real, cfg.d_model), generator=g, device=dev)
        bounds = torch.from_numpy(np.concatenate([np.stack([np.full(n, s), np.full(n, s + n)], axis=1)
                                                  for s, n in zip(starts, lengths)])).to(dev)
        keep = torch.from_numpy(np.concatenate([np.arange(n) + b * longest for b, n in enumerate(lengths)])).to(dev)
        xpad = torch.zeros((len(lengths) * longest, cfg.d_model), device=dev)
        xpad[keep] = xp.detach()
        xpad = xpad.view(len(lengths), longest, cfg.d_model).requires_grad_()
        wpad = torch.zeros((len(lengths) * longest, cfg.d_model), device=dev)
        wpad[keep] = wp
        wpad = wpad.view(len(lengths), longest, cfg.d_model)

        def ours_packed():
            with autocast:
                h = trunk(*trunk.condition(xp, None, None), bounds)
            (h * wp).sum().backward()

        def theirs_padded():
            with autocast:
                h = ref.forward_full(*ref.condition(xpad, None, None))
            (h * wpad).sum().backward()

        entry = {"sequences": len(lengths), "tokens": n_real, "padded_tokens": len(lengths) * longest,
                 "ms_per_step": round(wall(ours_packed) * 1e3, 3)}
        entry["tokens_per_s"] = round(n_real / entry["ms_per_step"] * 1e3, 1)
        if ref is not None:
            entry["reference_gpu_ms_per_step"] = round(wall(theirs_padded) * 1e3, 3)
            entry["speedup"] = round(entry["reference_gpu_ms_per_step"] / entry["ms_per_step"], 2)
        result["ragged_96_packed_vs_padded"] = entry
        trunk.zero_grad(set_to_none=True)
        out[precision] = result
    del trunk, ref
    torch.cuda.empty_cache()
    return out


def gemm_probe(device: torch.device, reps: int = 20) -> list:
    """The fp32 GEMMs of one training layer at 16384 tokens (d 256, d_ff 1024, QKV 384): the
    token-major products x W^T and the weight gradients dY^T X, ours beside torch.matmul."""

    from card_playing_gym_amd.nn import train as T

    n, out = 16384, []

    def run(fn) -> float:
        for _ in range(3):
            fn()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / reps * 1e3

    g = torch.Generator(device=device).manual_seed(3)
    for m, nn_, k in ((n, 1024, 256), (n, 256, 1024), (n, 256, 256), (n, 384, 256), (n, 256, 384)):
        x = torch.randn((m, k), generator=g, device=device)
        w = torch.randn((nn_, k), generator=g, device=device)
        y = torch.empty((m, nn_), device=device)
        ours, theirs = run(lambda: T.linear_nt(x, w, y)), run(lambda: torch.matmul(x, w.t(), out=y))
        out.append({"op": "x W^T", "m": m, "n": nn_, "k": k, "us": round(ours, 1), "torch_us": round(theirs, 1),
                    "tflops": round(2 * m * nn_ * k / ours / 1e6, 1)})
    for rows, cols in ((1024, 256), (256, 1024), (256, 256), (384, 256)):
        dy = torch.randn((n, rows), generator=g, device=device)
        x = torch.randn((n, cols), generator=g, device=device)
        y = torch.empty((rows, cols), device=device)
        ours, theirs = run(lambda: T.matmul_tn(dy, x, y)), run(lambda: torch.matmul(dy.t(), x, out=y))
        out.append({"op": "dY^T X", "m": rows, "n": cols, "k": n, "us": round(ours, 1), "torch_us": round(theirs, 1),
                    "tflops": round(2 * rows * cols * n / ours / 1e6, 1)})
    return out


def cpu_baseline(name: str, games: int, steps: int, first: int, horizon: int) -> dict:
    """The oracle's reference path on the host cores, on `games` of the workload's games, at
    steps first .. first + steps (the middle of the timed range: context lengths there are
    the timed region's average)."""

    from card_playing_gym_amd.synthetic import WORKLOADS, Driver, build_model
    from oracle.reference_path import RefCache, RefSynthetic, ref_config_of

    w = WORKLOADS[name]
    cores = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "1024")))
    torch.set_num_threads(cores)
    config = w.trunk_config()
    model = build_model(config, seed=0)
    state = {k: v.detach() for k, v in model.state_dict().items()}
    ref = RefSynthetic(state, ref_config_of(config), w.precision)
    small = type(w)(**{**w.__dict__, "games": games})
    driver = Driver(small, seed=0, max_len=w.max_len(horizon))
    max_len = driver.max_len
    for _ in range(first - 1):  # advance the host state (lengths) to the sampled steps
        driver.step()
    cache = RefCache(config.n_layers, config.n_kv_heads, config.head_dim, games, max_len, w.kv_dtype)
    times = []
    with torch.no_grad():
        for step in range(steps + 1):
            plan = driver.step()
            span = min(int(-(-(plan.positions.max() + 1) // 32) * 32), max_len)
            t0 = time.perf_counter()
            hidden = ref.forward_ragged(
                torch.from_numpy(plan.tokens).view(-1, 1, 1), torch.from_numpy(plan.positions), cache,
                torch.from_numpy(plan.readout), span=span,
                rows=torch.from_numpy(plan.rows) if w.mode == "continuous" else None,
            )
            ref.heads(hidden)
            times.append(time.perf_counter() - t0)
    per_step = float(np.mean(times[1:]))
    return {
        "value": round(games / per_step, 1),
        "unit": "game-tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{name} restated reference path (eager PyTorch CPU, {w.precision} rounding, {w.kv_dtype} KV): "
        f"{games} of the {w.games} games, 1 untimed + {steps} timed steps from step {first} (the middle of "
        f"the GPU's timed range), {per_step * 1e3:.0f} ms/step",
    }


def reference_gpu(bench: Bench, steps: int, first: int, compiled: bool = True) -> dict:
    """The restated reference path on the MI355X on steps first .. first + steps - 1 (the
    middle of the timed range), three ways: eager; captured in one graph; and as the
    reference's CUDA rollout runs it (cardgym/rl/graphs.py:66-151 with cardgym/nn/compile.py:
    26-44): torch.compile(dynamic=True), warmed up on a side stream, then captured and
    replayed.  span is what the reference's collector passes: the longest row after the
    append, rounded up to 32 (cardgym/rl/continuous.py:338), one value for the sampled steps
    (one graph shape).  Packed chunks run as the reference's collector pads them: repeat-last
    to the longest chunk (continuous.py:324-338)."""

    from oracle.reference_path import RefCache, RefSynthetic, ref_config_of

    w = bench.workload
    cfg = bench.config
    dev = bench.device
    state = {k: v.detach() for k, v in bench.model.state_dict().items()}
    ref = RefSynthetic(state, ref_config_of(cfg), w.precision)
    cache = RefCache(cfg.n_layers, cfg.n_kv_heads, cfg.head_dim, w.capacity(), bench.max_len, w.kv_dtype, device=dev)
    sampled = range(first, first + steps)
    run = max(int(np.diff(bench.plans[s].seq_start).max()) for s in sampled)
    tok = torch.zeros((bench.games, run, 1), dtype=torch.int64, device=dev)
    pos = torch.zeros(bench.games, dtype=torch.int64, device=dev)
    rows = torch.arange(bench.games, dtype=torch.int64, device=dev)
    readout = torch.zeros(bench.games, dtype=torch.int64, device=dev)
    last = max(int((bench.plans[s].positions + np.diff(bench.plans[s].seq_start)).max()) - 1 for s in sampled)
    span = min(int(-(-(last + 1) // 32) * 32), bench.max_len)
    padded = {}
    for s in sampled:
        plan = bench.plans[s]
        counts = np.diff(plan.seq_start)
        t = np.zeros((bench.games, run), dtype=np.int64)
        for b in range(bench.games):
            chunk = plan.tokens[plan.seq_start[b]:plan.seq_start[b + 1]]
            t[b, :chunk.size] = chunk
            t[b, chunk.size:] = chunk[-1]
        padded[s] = (torch.from_numpy(t).to(dev), torch.from_numpy(counts - 1).to(dev))
    gathered = bench.gathered
    game_tokens = bench.tokens_in(first, steps)

    def body(tok, pos, rows, readout):
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=False):
            hidden = ref.forward_ragged(tok, pos, cache, readout, span=span, rows=rows if gathered else None)
            return ref.heads(hidden)

    def load(step):
        tok.copy_(padded[step][0][..., None])
        readout.copy_(padded[step][1])
        pos.copy_(bench.positions_all[step])
        rows.copy_(bench.rows_all[step])

    def graphed(fn) -> float:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn(tok, pos, rows, readout)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn(tok, pos, rows, readout)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in sampled:
            load(s)
            graph.replay()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    result = {}
    with torch.no_grad():
        load(first)
        body(tok, pos, rows, readout)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in sampled:
            load(s)
            body(tok, pos, rows, readout)
        torch.cuda.synchronize()
        result["eager_game_tokens_per_s"] = round(game_tokens / (time.perf_counter() - t0), 1)
        result["graph_game_tokens_per_s"] = round(game_tokens / graphed(body), 1)
        if compiled:
            from torch import _dynamo
            from torch._inductor import config as inductor_config

            # The reference's settings (cardgym/nn/compile.py:35-44): compile in this process.
            inductor_config.compile_threads = 1
            _dynamo.config.cache_size_limit = max(_dynamo.config.cache_size_limit, 64)
            _dynamo.reset()
            try:
                load(first)
                t0 = time.perf_counter()
                fn = torch.compile(body, dynamic=True)
                fn(tok, pos, rows, readout)
                torch.cuda.synchronize()
                result["compile_s"] = round(time.perf_counter() - t0, 1)
                result["compiled_graph_game_tokens_per_s"] = round(game_tokens / graphed(fn), 1)
            except Exception as exc:  # recorded, not hidden: the leg stays in the line
                result["compiled_graph_error"] = f"{type(exc).__name__}: {str(exc)[:300]}"
            _dynamo.reset()
        result["span"] = span
        result["steps"] = f"{first}..{first + steps - 1}"
    del cache
    torch.cuda.empty_cache()
    return result


def best_reference(result: dict) -> float:
    """The fastest of the reference path's legs (eager, graph, compiled + graph)."""

    legs = ("eager_game_tokens_per_s", "graph_game_tokens_per_s", "compiled_graph_game_tokens_per_s")
    return max(result[k] for k in legs if k in result)


def projections(bench: Bench, step_s: float, attention: dict, n_tokens: float) -> dict:
    """MFMA throughput of the step's bf16 projections (QKV, out, MLP up / down; the fused
    layer kernels), from the whole step's time less its attention launches: the rest also
    holds the embedding, plan, final norm and heads launches (tens of microseconds), so this
    bounds the projections' rate from below."""

    from card_playing_gym_amd.synthetic import projection_flops

    flops = projection_flops(bench.config, 1) * n_tokens
    rest = step_s - attention["avg_launch_us"] * 1e-6 * bench.config.n_layers
    tflops = flops / rest / 1e12
    return {"flops_per_step": int(flops), "step_less_attention_us": round(rest * 1e6, 1),
            "tflops_lower_bound": round(tflops, 1), "peak_tflops": 2500.0,
            "frac_lower_bound": round(tflops / 2500.0, 4)}


def time_steps(bench: Bench, first: int, count: int) -> float:
    """Wall seconds of `count` graph-replayed steps from `first`, device-synchronised on
    both sides (and the HIP-event span, whichever is longer)."""

    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for s in range(first, first + count):
        bench.step(s)
    end.record()
    torch.cuda.synchronize()
    return max(time.perf_counter() - t0, start.elapsed_time(end) / 1e3)


def workload_line(name: str, steps: int, warmup: int, ref_steps: int, with_reference: bool) -> dict:
    """Config 4 or 5 beside the headline: game-tokens/s over `steps` graph-replayed steps after
    `warmup`, the attention roofline of the same steps, the projections' rate, and the
    restated reference path on the same GPU (eager, graph, compiled + graph)."""

    bench = Bench(name, steps, warmup)
    w = bench.workload
    with torch.no_grad():
        bench.load(0)
        bench.capture(tuple(range(warmup + steps)) if bench.chunks else (0,))
        for s in range(warmup):
            bench.step(s)
        elapsed = time_steps(bench, warmup, steps)
    game_tokens = bench.tokens_in(warmup, steps)
    out = {
        "workload": f"{w.name}: {w.description}",
        "game_tokens_per_s": round(game_tokens / elapsed, 1),
        "ms_per_step": round(elapsed / steps * 1e3, 4),
        "tokens_per_step": round(game_tokens / steps, 1),
        "steps": steps,
        "warmup": warmup,
        "max_len": bench.max_len,
    }
    if w.mode == "continuous":
        out["games_ended_per_step"] = round(sum(int((bench.plans[s + 1].positions == 0).sum())
                                                for s in range(warmup, warmup + steps - 1)) / (steps - 1), 1)
    with torch.no_grad():
        out["roofline"] = attention_roofline(bench, warmup, steps)
    out["projections"] = projections(bench, elapsed / steps, out["roofline"], game_tokens / steps)
    if with_reference:
        middle = warmup + steps // 2 - ref_steps // 2
        ref = reference_gpu(bench, ref_steps, middle)
        # The reference's rate on its sampled steps, ours on the same steps.
        with torch.no_grad():
            ours = bench.tokens_in(middle, ref_steps) / time_steps(bench, middle, ref_steps)
        ref["ours_same_steps_game_tokens_per_s"] = round(ours, 1)
        ref["speedup_vs_best"] = round(ours / best_reference(ref), 2)
        out["reference_gpu"] = ref
    bench.graphs.clear()
    bench.graph = None
    del bench
    torch.cuda.empty_cache()
    return out


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the decode step has no "
            "cross-GPU exchange; games shard across GPUs with replicated weights, see DESIGN.md).",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    torch.backends.cuda.matmul.allow_tf32 = False
    log(f"bench: setting up {args.workload} ({args.warmup} warmup + {args.steps} timed steps)")
    if args.gemm_probe:  # needs no workload state
        print(json.dumps({"probe": "gemm", "shapes": gemm_probe(torch.device("cuda", 0))}), flush=True)
        return 0
    bench = Bench(args.workload, args.steps, args.warmup)
    w = bench.workload
    if args.traffic_probe:
        # Counter passes read per-dispatch HBM traffic: the attention launches of the timed
        # steps (as the roofline replays them) and a plain device copy of known size, whose
        # reading calibrates the counters.
        with torch.no_grad():
            roof = attention_roofline(bench, args.warmup, args.steps)
            src = torch.ones(256 << 20, dtype=torch.uint8, device=bench.device)
            dst = torch.empty_like(src)
            for _ in range(4):
                dst.copy_(src)
            torch.cuda.synchronize()
        print(json.dumps({"probe": "traffic", "kernel": roof["kernel"], "launches": roof["launches"],
                          "algorithmic_bytes_per_launch": roof["algorithmic_bytes_per_launch"],
                          "copy_bytes": src.numel(), "copy_launches": 4}), flush=True)
        return 0
    if args.train_probe:
        print(json.dumps({"probe": "train_step", **train_step_time(bench, with_reference=False)}), flush=True)
        return 0
    if args.compaction_probe:
        with torch.no_grad():
            print(json.dumps({"probe": "compaction", **compaction_time(bench)}), flush=True)
        return 0
    with torch.no_grad():
        bench.load(0)
        bench.capture(tuple(range(args.warmup + args.steps)) if bench.chunks else (0,))
        if args.step_probe:
            for s in range(args.warmup):
                bench.step(s)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for s in range(args.warmup, args.warmup + args.steps):
                bench.step(s)
            torch.cuda.synchronize()
            per_step = (time.perf_counter() - t0) / args.steps
            print(json.dumps({"probe": "step", "workload": args.workload, "steps": args.steps, "warmup": args.warmup,
                              "ms_per_step": round(per_step * 1e3, 4),
                              "game_tokens_per_s": round(bench.tokens_in(args.warmup, args.steps) / args.steps / per_step, 1)}),
                  flush=True)
            return 0
        torch.cuda.synchronize()
        for s in range(args.warmup):
            bench.step(s)
        torch.cuda.synchronize()
        log("bench: warmup done, timing")
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for s in range(args.warmup, args.warmup + args.steps):
            bench.step(s)
        end.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    elapsed = max(wall, start.elapsed_time(end) / 1e3)
    tokens = bench.tokens_in(args.warmup, args.steps)
    value = tokens / elapsed
    log(f"bench: {value:,.0f} game-tokens/s, {elapsed / args.steps * 1e3:.3f} ms/step")
    with torch.no_grad():
        roofline = attention_roofline(bench, args.warmup, args.steps)
    log(f"bench: decode attention {roofline['achieved']:.0f} GB/s ({roofline['frac']:.1%} of peak), "
        f"{roofline['avg_launch_us']} us/launch")
    extra = {"projections": projections(bench, elapsed / args.steps, roofline, tokens / args.steps)}
    log(f"bench: projections {extra['projections']}")
    extra["sampling"] = sampling_time(bench)
    log(f"bench: device sampling {extra['sampling']}")
    cpu = None
    middle = args.warmup + args.steps // 2 - args.ref_steps // 2
    if not args.no_baselines:
        ref = reference_gpu(bench, args.ref_steps, middle)
        with torch.no_grad():
            ref["ours_same_steps_game_tokens_per_s"] = round(
                bench.tokens_in(middle, args.ref_steps) / time_steps(bench, middle, args.ref_steps), 1)
        ref["speedup_vs_best"] = round(value / best_reference(ref), 2)
        ref["speedup_same_steps_vs_best"] = round(ref["ours_same_steps_game_tokens_per_s"] / best_reference(ref), 2)
        extra["reference_gpu"] = ref
        log(f"bench: reference path on the GPU {extra['reference_gpu']}")
    # These rewrite cache rows: after everything that reads them.
    extra["compaction"] = compaction_time(bench)
    log(f"bench: compaction {extra['compaction']}")
    extra["prefill"] = prefill_time(bench, with_reference=not args.no_baselines)
    log(f"bench: prefill {extra['prefill']}")
    extra["piquet_embed"] = piquet_embed_time(bench.device, with_reference=not args.no_baselines)
    log(f"bench: piquet embedder {extra['piquet_embed']}")
    extra["piquet_wave"] = piquet_wave_time(bench, with_reference=not args.no_baselines)
    log(f"bench: piquet wave {extra['piquet_wave']}")
    extra["train_step"] = train_step_time(bench, with_reference=not args.no_baselines)
    log(f"bench: training step {extra['train_step']}")
    bench.graph = None
    del bench.cache
    torch.cuda.empty_cache()
    if not args.no_workloads:
        # Configs 4 and 5 at full size, each beside the reference path on the same GPU.
        for name in ("cfg4", "cfg5"):
            if name == args.workload:
                continue
            extra[name] = workload_line(name, args.steps, args.warmup, args.ref_steps, not args.no_baselines)
            log(f"bench: {name} {extra[name]}")
    if not args.no_baselines:
        cpu = cpu_baseline(args.workload, args.cpu_games, args.cpu_steps, middle, args.warmup + args.steps)
        log(f"bench: cpu baseline {cpu}")
    result = {
        "metric": "game-tokens/sec at 4096 games; decode-attn HBM GB/s vs peak",
        "value": round(value, 1),
        "unit": "game-tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, seed 0; token ids U[0,512); random initial KV prefixes)",
        "config": {
            "workload": f"{w.name}: {w.description}",
            "games": w.games,
            "layers": w.n_layers,
            "d_model": 256,
            "heads": "8/2",
            "head_dim": 32,
            "kv_dtype": str(w.kv_dtype).replace("torch.", ""),
            "max_len": bench.max_len,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(result), flush=True)
    _stop_compile_workers()
    return 0


def _descendants() -> list[int]:
    """PIDs of every process this one started, directly or not (from /proc)."""

    parent: dict[int, int] = {}
    for entry in os.listdir("/proc"):
        if not entry.isdigit():
            continue
        try:
            with open(f"/proc/{entry}/stat") as f:
                fields = f.read().rsplit(")", 1)[1].split()
            parent[int(entry)] = int(fields[1])
        except (OSError, IndexError, ValueError):
            continue
    found, frontier = [], [os.getpid()]
    while frontier:
        pid = frontier.pop()
        kids = [p for p, pp in parent.items() if pp == pid]
        found.extend(kids)
        frontier.extend(kids)
    return found


def _alive(pid: int) -> bool:
    try:
        with open(f"/proc/{pid}/stat") as f:
            return f.read().rsplit(")", 1)[1].split()[0] != "Z"
    except (OSError, IndexError):
        return False


def _stop_compile_workers() -> None:
    """The compiled reference leg starts Inductor's compile workers (a sidecar process and
    its pool) and multiprocessing may start a resource tracker: ask the workers to shut down,
    then wait for every process this one started, directly or through them, and end any
    that is still running after a grace period, so that no process outlives the benchmark.
    The descendants are listed before the shutdown, so that pool processes whose parent
    exits first are still waited for."""

    kids = _descendants()
    try:
        from torch._inductor.async_compile import shutdown_compile_workers
    except ImportError:
        shutdown_compile_workers = None
    if shutdown_compile_workers is not None:
        shutdown_compile_workers()
    for sig, grace in ((None, 3.0), (signal.SIGTERM, 3.0), (signal.SIGKILL, 2.0)):
        alive = [p for p in kids if _alive(p)]
        if not alive:
            break
        if sig is not None:
            for pid in alive:
                try:
                    os.kill(pid, sig)
                except OSError:
                    pass
        deadline = time.monotonic() + grace
        while time.monotonic() < deadline and any(_alive(p) for p in alive):
            for pid in alive:
                try:
                    os.waitpid(pid, os.WNOHANG)  # reaps direct children
                except ChildProcessError:
                    pass
            time.sleep(0.05)
    left = [p for p in kids if _alive(p)]
    if left:
        log(f"bench: {len(left)} child processes still running at exit")


if __name__ == "__main__":
    sys.exit(main())
