"""Worker processes that each own a device context, as the reference's asynchronous rollout
runs its collectors (cardgym/rl/async_rollout.py:147-165: one process per worker, each with
its own model copy and KV pool on the same GPU).

Two spawned workers load the library, build the model and a pool on the one GPU and step
the same seeded workload at the same time; each checks its steps against the oracle on its
own host copy of the pool (2e-2, bf16), and both must produce the same hidden states (the
library holds no state shared between processes).
"""

from __future__ import annotations

import multiprocessing as mp
import queue

import numpy as np
import pytest

from tests.workers import step_worker

pytestmark = pytest.mark.gpu

WORKERS = 2


def test_workers_step_concurrently_on_one_gpu(device):
    ctx = mp.get_context("spawn")
    results = ctx.Queue()
    procs = [ctx.Process(target=step_worker, args=(rank, results), daemon=True) for rank in range(WORKERS)]
    for proc in procs:
        proc.start()
    got = {}
    try:
        for _ in range(WORKERS):
            rank, worst, outputs, error = results.get(timeout=240)
            assert error is None, f"worker {rank}: {error}"
            print(f"worker {rank}: worst error {worst:.3g}", flush=True)
            assert worst <= 2e-2
            got[rank] = outputs
    except queue.Empty:
        pytest.fail("a worker did not report within 240 s")
    finally:
        for proc in procs:
            proc.join(timeout=60)
            if proc.is_alive():
                proc.terminate()
                proc.join(timeout=10)
    assert all(proc.exitcode == 0 for proc in procs)
    np.testing.assert_array_equal(got[0], got[1])
