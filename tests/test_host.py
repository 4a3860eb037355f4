"""Host-side tests (no GPU): the C ABI library, its argument checking, the Python mirror of
the cardgym.nn API and the workload drivers."""

from __future__ import annotations

import ctypes
import shutil
import subprocess
import sys
import textwrap

import numpy as np
import pytest
import torch

from card_playing_gym_amd import _native as nat
from card_playing_gym_amd.nn import KVCache, Trunk, TrunkConfig
from card_playing_gym_amd.synthetic import WORKLOADS, Driver, StepPlan, build_model, kv_bytes, trunk_config
from tests.conftest import ROOT


def test_library_exports_every_declared_symbol():
    lib = nat.lib()
    declared = nat.declared_symbols()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/cardgym_hip.h but not exported"
    assert set(declared) == set(nat._SIGNATURES), "ctypes signatures and header disagree"
    assert lib.cg_version() >= 100


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_struct_layouts_match_the_header(tmp_path):
    structs = {
        "cg_kv_layer": nat.KVLayer,
        "cg_kv_source": nat.KVSource,
        "cg_trunk_config": nat.TrunkConfig,
        "cg_layer_params": nat.LayerParams,
        "cg_ragged": nat.Ragged,
    }
    lines = []
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    source = tmp_path / "layout.c"
    source.write_text(
        "#include <stdio.h>\n#include <stddef.h>\n#include \"cardgym_hip.h\"\nint main(void){\n"
        + "\n".join(lines)
        + "\nreturn 0;}\n"
    )
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(source), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    for line in filter(None, out):
        cname, field, value = line.split()
        py = structs[cname]
        expected = ctypes.sizeof(py) if field == "size" else getattr(py, field).offset
        assert int(value) == expected, f"{cname}.{field}: C {value} vs ctypes {expected}"


def test_argument_errors_come_back_as_status_and_message():
    lib = nat.lib()
    assert lib.cg_kv_write_step(None, None, None, None, None, 1, 1, None) == nat.CG_ERR_INVALID
    assert "positions is NULL" in nat.last_error()
    with pytest.raises(ValueError, match="cache layer is NULL"):
        nat.call("cg_kv_write_range", None, None, 0, None, None, 1, 1, None)

    layer = nat.KVLayer(16, 16, 4, 2, 8, 40, nat.CG_F32)  # fake pointers: never dereferenced
    status = lib.cg_decode_attention(16, nat.CG_F32, 0, 0, 0, ctypes.byref(layer), None, 16, 1, 4, 1, 0, 1.0, 16,
                                     nat.CG_F32, None)
    assert status == nat.CG_ERR_UNSUPPORTED and "head_dim" in nat.last_error()
    bad_dtype = nat.KVLayer(16, 16, 4, 2, 8, 32, 7)
    assert lib.cg_kv_read(ctypes.byref(bad_dtype), None, 1, 1, 16, 16, None) == nat.CG_ERR_INVALID
    layer32 = nat.KVLayer(16, 16, 4, 2, 8, 32, nat.CG_F32)
    assert lib.cg_kv_read(ctypes.byref(layer32), None, 1, 9, 16, 16, None) == nat.CG_ERR_RANGE
    with pytest.raises(IndexError):
        nat.call("cg_kv_read", ctypes.byref(layer32), None, 1, 9, 16, 16, None)

    assert lib.cg_linear(16, 16, None, 16, 4, 4, 12, nat.CG_ACT_NONE, nat.CG_F32, None) == nat.CG_ERR_UNSUPPORTED
    assert lib.cg_linear(16, 16, None, 16, 4, 4, 16, 9, nat.CG_F32, None) == nat.CG_ERR_INVALID
    assert lib.cg_trunk_workspace_size(None, 4, 4) == 0


def _create(config: nat.TrunkConfig, compute=nat.CG_F32) -> int:
    layers = (nat.LayerParams * max(config.n_layers, 1))()
    for i in range(max(config.n_layers, 1)):
        layers[i] = nat.LayerParams(*([16] * 10), -1)
    handle = ctypes.c_void_p()
    return nat.lib().cg_trunk_create(ctypes.byref(config), layers, 16, 16, compute, ctypes.byref(handle))


def test_trunk_create_validates_the_config():
    assert _create(nat.TrunkConfig(250, 2, 8, 2, 1024, 0, 0, 1e-5)) == nat.CG_ERR_INVALID  # 250 % 8
    assert "divisible" in nat.last_error()
    assert _create(nat.TrunkConfig(256, 2, 8, 3, 1024, 0, 0, 1e-5)) == nat.CG_ERR_INVALID
    assert _create(nat.TrunkConfig(320, 2, 8, 2, 1024, 0, 0, 1e-5)) == nat.CG_ERR_UNSUPPORTED  # head_dim 40
    assert _create(nat.TrunkConfig(256, 2, 8, 2, 1024, 0, 0, 1e-5), compute=nat.CG_F16) == nat.CG_ERR_INVALID


def test_trunk_forward_checks_its_step_before_launching():
    lib = nat.lib()
    handle = ctypes.c_void_p()
    config = nat.TrunkConfig(256, 1, 8, 2, 1024, 0, 0, 1e-5)
    layers = (nat.LayerParams * 1)(nat.LayerParams(*([16] * 10), -1))
    assert lib.cg_trunk_create(ctypes.byref(config), layers, 16, 16, nat.CG_F32, ctypes.byref(handle)) == 0
    try:
        need = lib.cg_trunk_workspace_size(handle, 64, 64)
        assert need >= 64 * 256 * 4 * 2
        cache = (nat.KVLayer * 1)(nat.KVLayer(16, 16, 64, 2, 32, 32, nat.CG_BF16))
        step = nat.Ragged(64, 64, 1, 0, None, 16, None, 16)
        # Too small a workspace is refused before anything is enqueued.
        assert lib.cg_trunk_forward(handle, cache, 16, None, None, ctypes.byref(step), 16, 16, need - 1, None) == 1
        assert "workspace too small" in nat.last_error()
        wrong = (nat.KVLayer * 1)(nat.KVLayer(16, 16, 64, 4, 32, 32, nat.CG_BF16))
        assert lib.cg_trunk_forward(handle, wrong, 16, None, None, ctypes.byref(step), 16, 16, need, None) == 1
        assert "does not match" in nat.last_error()
        mismatch = nat.Ragged(64, 65, 1, 0, None, 16, None, 16)
        assert lib.cg_trunk_forward(handle, cache, 16, None, None, ctypes.byref(mismatch), 16, 16, need, None) == 1
        dense = nat.Ragged(65, 65, 1, 0, None, 16, None, 16)
        assert lib.cg_trunk_forward(handle, cache, 16, None, None, ctypes.byref(dense), 16, 16, need * 2, None) == nat.CG_ERR_RANGE
    finally:
        assert lib.cg_trunk_destroy(handle) == 0


def test_heads_create_validates_the_config():
    lib = nat.lib()
    handle = ctypes.c_void_p()

    def create(*cfg):
        config = nat.HeadsConfig(*cfg)
        return lib.cg_heads_create(ctypes.byref(config), 16, 16, 16, 16, 16, 16, ctypes.byref(handle))

    # Shapes outside the fused kernel are refused before any device call.
    assert create(250, 512, 256, 2) == nat.CG_ERR_UNSUPPORTED  # d_model % 16
    assert "multiples of 16" in nat.last_error()
    assert create(288, 512, 256, 2) == nat.CG_ERR_UNSUPPORTED  # d_model > 256
    assert create(256, 1040, 256, 2) == nat.CG_ERR_UNSUPPORTED  # n_policy > 1024
    assert create(256, 520, 256, 2) == nat.CG_ERR_UNSUPPORTED  # n_policy % 16
    assert create(256, 512, 272, 2) == nat.CG_ERR_UNSUPPORTED  # d_mid > 256
    assert create(256, 512, 256, 0) == nat.CG_ERR_UNSUPPORTED
    assert create(256, 512, 256, 17) == nat.CG_ERR_UNSUPPORTED
    config = nat.HeadsConfig(256, 512, 256, 2)
    assert lib.cg_heads_create(ctypes.byref(config), None, 16, 16, 16, 16, 16, ctypes.byref(handle)) == nat.CG_ERR_INVALID
    assert lib.cg_heads_forward(None, 16, 4, 16, 16, None) == nat.CG_ERR_INVALID
    assert lib.cg_heads_destroy(None) == 0


def test_sampling_entry_points_check_their_arguments():
    lib = nat.lib()
    assert lib.cg_masked_probabilities(16, 4, 16, 4, -1, 4, 16, 4, None) == nat.CG_ERR_INVALID
    assert lib.cg_masked_probabilities(16, 3, 16, 4, 2, 4, 16, 4, None) == nat.CG_ERR_INVALID  # stride < width
    assert lib.cg_masked_probabilities(None, 4, 16, 4, 2, 4, 16, 4, None) == nat.CG_ERR_INVALID
    assert lib.cg_masked_probabilities(None, 4, None, 4, 0, 4, None, 4, None) == 0  # nothing to do
    assert lib.cg_sample_rows(16, 4, 16, 4, 16, 2, 0, 16, None) == nat.CG_ERR_INVALID  # width 0
    assert lib.cg_sample_rows(16, 4, None, 4, 16, 2, 4, 16, None) == nat.CG_ERR_INVALID


def test_trunk_config_matches_the_reference_rules():
    assert TrunkConfig(n_layers=16, value_embeddings="alternating").value_layers == tuple(range(1, 16, 2))
    assert TrunkConfig(n_layers=5, value_embeddings="alternating").value_layers == (0, 2, 4)
    assert TrunkConfig(n_layers=3, value_embeddings="all").value_layers == (0, 1, 2)
    cfg = TrunkConfig(d_model=240, n_layers=16, n_heads=10, n_kv_heads=2, per_layer_dim=64, value_embeddings="alternating")
    assert (cfg.head_dim, cfg.kv_width, cfg.ple_width, cfg.value_width) == (24, 48, 1024, 8 * 48)
    with pytest.raises(ValueError):
        TrunkConfig(d_model=250, n_heads=8).validate()
    with pytest.raises(ValueError):
        TrunkConfig(n_heads=8, n_kv_heads=3).validate()


def test_parameter_names_match_the_reference_state_dict():
    trunk = Trunk(TrunkConfig(d_model=32, n_layers=2, n_heads=4, n_kv_heads=2, d_ff=64, per_layer_dim=8))
    keys = set(trunk.state_dict())
    expected = {"input_norm.weight", "ple_context.weight", "final_norm.weight", "final_norm.bias"}
    for i in range(2):
        expected |= {
            f"blocks.{i}.{name}"
            for name in ("ln_attn.weight", "ln_attn.bias", "qkv_proj.weight", "out_proj.weight", "ln_mlp.weight",
                         "ln_mlp.bias", "mlp.0.weight", "mlp.0.bias", "mlp.2.weight", "mlp.2.bias")
        }
    assert keys == expected
    assert trunk.blocks[0].qkv_proj.weight.shape == (4 * 8 + 2 * 2 * 8, 32)
    assert float(trunk.ple_context.weight.detach().abs().sum()) == 0.0  # conditioning starts at zero
    # GPT-2 residual scaling of out_proj and mlp[2] (std 0.02 / sqrt(2 * n_layers)).
    big = Trunk(TrunkConfig(d_model=256, n_layers=8, n_heads=8, n_kv_heads=2, d_ff=1024))
    assert abs(big.blocks[0].out_proj.weight.std().item() - 0.02 / 4) < 5e-4
    assert abs(big.blocks[0].qkv_proj.weight.std().item() - 0.02) < 5e-4


def test_kv_cache_host_behaviour():
    cache = KVCache(n_layers=2, kv_heads=2, head_dim=8, capacity=3, max_len=5, device="cpu", dtype=torch.bfloat16)
    assert cache.stacked and cache.k[1].shape == (3, 2, 5, 8) and cache.k[1].dtype == torch.bfloat16
    assert cache.k[1].data_ptr() == cache._base_k[1].data_ptr()
    assert KVCache.bytes_per_row(16, 2, 32, 769, torch.bfloat16) == 16 * 2 * 769 * 32 * 2 * 2
    k, _ = cache.read(0, None, 3, count=2)
    assert k.shape == (2, 2, 3, 8) and k.data_ptr() == cache.k[0].data_ptr()
    with pytest.raises(ValueError, match="explicit row count"):
        cache.read(0, None, 3)
    with pytest.raises(RuntimeError, match="ROCm GPU only"):
        cache.write_step(0, torch.tensor([0]), torch.tensor([1]), torch.zeros(1, 2, 1, 8), torch.zeros(1, 2, 1, 8))
    with pytest.raises(ValueError):
        KVCache(n_layers=1, kv_heads=1, head_dim=8, capacity=1, max_len=4, device="cpu", dtype=torch.int8)


def test_model_exposes_what_the_reference_trainer_reads():
    """The reference's trainer and setup read model.packs(device) on every microbatch
    (cardgym/rl/trainer.py:659), trunk.metal / trunk.uses_metal(...) to pick its MPS-only fused
    trunk (trainer.py:709, setup.py:142) and call model.enable_metal_trunk (setup.py:111): the
    HIP model answers them without a Metal trunk, and packs rows on the ROCm GPU only."""

    from card_playing_gym_amd.nn import SequenceModel

    model = SequenceModel(TrunkConfig(d_model=64, n_layers=1, n_heads=4, n_kv_heads=2, d_ff=128))
    assert model.trunk.metal is None
    assert model.trunk.uses_metal(torch.device("cuda", 0), 128) is False
    assert model.packs(torch.device("cpu")) is False
    assert model.packs(torch.device("cuda", 0)) is (torch.version.hip is not None)
    assert model.enable_metal_trunk(512) is None and model.trunk.metal is None
    for name in ("forward_ragged", "forward_prefill", "final_norm", "config", "condition"):
        assert hasattr(model.trunk, name), name


def test_no_cpu_fallback_in_the_product_path():
    model = build_model(TrunkConfig(d_model=64, n_layers=1, n_heads=4, n_kv_heads=2, d_ff=128))
    tokens = torch.zeros((2, 1, 1), dtype=torch.int64)
    cache = model.new_cache(2, 4)
    with pytest.raises(RuntimeError, match="ROCm GPU only"):
        model.forward_ragged(tokens, torch.zeros(2, dtype=torch.int64), cache, torch.zeros(2, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="ROCm GPU only"):
        model.forward_hidden(tokens)


def test_workload_drivers_are_deterministic_and_well_formed():
    for name in WORKLOADS:
        w = WORKLOADS[name]
        small = type(w)(**{**w.__dict__, "games": 64})
        a, b = Driver(small, seed=0, max_len=2048), Driver(small, seed=0, max_len=2048)
        for _ in range(5):
            pa, pb = a.step(), b.step()
            for field in ("tokens", "positions", "rows", "seq_start", "readout"):
                assert np.array_equal(getattr(pa, field), getattr(pb, field))
            counts = np.diff(pa.seq_start)
            assert pa.seq_start[0] == 0 and (counts >= 1).all() and (counts <= w.max_chunk).all()
            assert np.array_equal(pa.readout, counts - 1)
            assert np.array_equal(np.sort(pa.rows), np.arange(64))
            assert ((pa.tokens >= 0) & (pa.tokens < 512)).all()


def test_continuous_workload_resets_slots():
    w = WORKLOADS["cfg4"]
    small = type(w)(**{**w.__dict__, "games": 2000})
    driver = Driver(small, seed=0, max_len=2048)
    assert abs(driver.lengths.mean() - 199) < 15  # stationary Geometric(1/200) ages
    prev = driver.lengths.copy()
    plan = driver.step()
    assert np.array_equal(plan.positions, prev[plan.rows])
    grown = driver.lengths == prev + 1
    reset = driver.lengths == 0
    assert (grown | reset).all() and 0 < reset.sum() < 40
    assert not np.array_equal(plan.rows, np.arange(2000))


def test_kv_bytes_counts_each_prefix_once():
    plan = StepPlan(np.zeros(5, dtype=np.int64), np.array([3, 0]), np.array([0, 1]), np.array([0, 2, 5]), np.array([1, 2]))
    # game 0: 3 cached + 2 new keys, game 1: 0 + 3; x 2 heads x 32 dims x (K, V) x 2 bytes x 4 layers
    assert kv_bytes(plan, 4, 2, 32, 2) == (5 + 3) * 2 * 32 * 2 * 2 * 4


def test_bench_refuses_more_than_one_gpu():
    result = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True)
    assert result.returncode == 2 and "one GPU" in result.stderr


def test_workload_shapes_match_the_benchmark_configs():
    assert WORKLOADS["cfg3"].games == 4096 and WORKLOADS["cfg3"].n_layers == 16
    assert WORKLOADS["cfg3"].kv_dtype == torch.bfloat16 and (WORKLOADS["cfg3"].length_low, WORKLOADS["cfg3"].length_high) == (1, 512)
    assert WORKLOADS["cfg1"].games == 64 and WORKLOADS["cfg1"].max_len(128) == 129
    assert WORKLOADS["cfg4"].games == 8192 and WORKLOADS["cfg5"].max_chunk == 16
    cfg = trunk_config(16)
    assert (cfg.d_model, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.d_ff) == (256, 8, 2, 32, 1024)
    assert textwrap.dedent("x") == "x"


def test_ordered_pairs_matches_its_definition():
    """ordered_pairs: every row in the pool and no pair i writes a row that a later pair k
    reads (t_i == s_k, i < k) -- checked against that definition by brute force, and
    against its consequence: copying the pairs in order equals gathering them first."""

    from card_playing_gym_amd.nn.kv_cache import ordered_pairs

    rng = np.random.default_rng(3)
    seen = {True: 0, False: 0}
    for _ in range(400):
        cap = int(rng.integers(1, 12))
        n = int(rng.integers(0, 8))
        s = rng.integers(-1 if rng.random() < 0.1 else 0, cap + (1 if rng.random() < 0.1 else 0), n)
        t = rng.permutation(cap)[: min(n, cap)] if rng.random() < 0.7 else rng.integers(0, cap, n)
        s = s[: t.size]
        got = ordered_pairs(s, t, cap)
        inside = all(0 <= x < cap for x in list(s) + list(t))
        brute = inside and not any(t[i] == s[k] for i in range(s.size) for k in range(i + 1, s.size))
        assert got == brute, (s, t, cap)
        seen[got] += 1
        if got:
            rows = np.arange(cap) * 10 + 7
            gathered = rows.copy()
            gathered[t] = rows[s]
            walked = rows.copy()
            for i in range(s.size):
                walked[t[i]] = walked[s[i]]
            if len(set(t.tolist())) == t.size:  # duplicate targets have no defined order
                assert (walked == gathered).all()
    assert seen[True] > 50 and seen[False] > 50
    # Compaction (rows slide down) is ordered; a swap and a shift up are not.
    assert ordered_pairs(np.array([3, 4, 5, 9]), np.array([0, 1, 2, 3]), 10)
    assert not ordered_pairs(np.array([1, 2]), np.array([2, 1]), 4)
    assert not ordered_pairs(np.array([0, 1, 2]), np.array([1, 2, 3]), 4)


def test_packed_bounds_to_sequence_starts():
    """Packed-row bounds as cardgym.nn.packing.Packing builds them (packing.py:24-40: int32
    [N, 2], row i -> [start, end) of its sequence) give the sequences' starts and the longest
    one; bounds that do not tile the rows with whole sequences are refused."""

    lengths = np.array([3, 1, 5, 2])
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    first = np.repeat(starts, lengths)
    bounds = torch.from_numpy(np.stack([first, first + np.repeat(lengths, lengths)], axis=1).astype(np.int32))
    seq_start, longest = Trunk._seq_start_of(bounds)
    assert seq_start.dtype == torch.int64 and seq_start.tolist() == [0, 3, 4, 9, 11] and longest == 5
    assert Trunk._seq_start_of(torch.tensor([[0, 1]], dtype=torch.int32))[0].tolist() == [0, 1]

    short_end = bounds.clone()
    short_end[2, 1] -= 1  # the first sequence's last row ends one row early
    split_seq = bounds.clone()
    split_seq[5:9, 0] = 5  # the third sequence's rows claim a start inside it
    for bad in (short_end, split_seq):
        with pytest.raises(ValueError, match="back to back"):
            Trunk._seq_start_of(bad)
    with pytest.raises(ValueError, match=r"\[N, 2\]"):
        Trunk._seq_start_of(bounds[:, :1])
    with pytest.raises(ValueError, match="at least one row"):
        Trunk._seq_start_of(bounds[:0])
