"""Worker body of tests/test_gpu_workers.py (a module of its own, so that spawned workers
import it by name)."""

from __future__ import annotations

import numpy as np

STEPS = 3


def step_worker(rank: int, results) -> None:
    # A fresh interpreter (spawn): everything it needs is imported here.
    try:
        import torch

        from card_playing_gym_amd.synthetic import Driver, Workload
        from tests.helpers import cache_pair, max_err, run_native, run_oracle, twins

        device = torch.device("cuda", 0)
        workload = Workload("workers", 4, 96, torch.bfloat16, "bf16", "continuous", 1, 200,
                            max_len_cap=320, end_probability=0.1)
        config = workload.trunk_config()
        model, ref = twins(config, "bf16", device, seed=7)
        max_len = workload.max_len(STEPS)
        driver = Driver(workload, seed=11, max_len=max_len)
        native, oracle = cache_pair(config, workload.capacity(), max_len, torch.bfloat16, device)
        worst, outputs = 0.0, []
        for _ in range(STEPS):
            plan = driver.step()
            hidden, _, _ = run_native(model, native, plan, device, "bf16", False, True)
            r_hidden, _, _ = run_oracle(ref, oracle, plan, True)
            worst = max(worst, max_err(hidden, r_hidden))
            outputs.append(hidden.float().cpu().numpy())
        native.check()
        results.put((rank, worst, np.stack(outputs), None))
    except BaseException as error:  # reported to the parent, which fails the test
        results.put((rank, None, None, repr(error)))
