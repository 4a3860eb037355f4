"""Writes the golden vectors of this folder by running the reference's own modules.

Run in the build container only, where the reference tree exists (it never travels to
the GPU box; only the .npz files this writes do):

    python tests/golden/make_golden.py [--reference /root/reference]

It imports, from the reference tree, the modules that hold what no closed form,
invariant or library routine pins:

* ``trunk_ragged_bf16kv.npz`` -- ``Trunk.condition`` + ``Trunk.forward_ragged``
  (cardgym/nn/trunk.py:285-312, 391-429) over a bf16 ``KVCache`` (kv_cache.py:19-138) with
  fp32 weights and no autocast: the rounding chain of trunk.py:222, 245 and 255 (q cast to
  the cache dtype, bf16 scores and scale, fp32 softmax cast back to bf16, bf16 P @ V).
  Two steps on a cfg1-shaped trunk (8 layers, d_model 256, 8 / 2 heads, d_ff 1024):
    - ``step1``: one token per game, gathered rows (a permutation of the pool's rows), one
      game restarted at length 0 over a previous game's stale prefix (slot reuse,
      cardgym/rl/continuous.py:232-261);
    - ``chunk``: a padded run of four tokens per game with 1-4 real ones (repeat-last
      padding, continuous.py:324-338), rows whose padding is clamped onto the reserved
      last slot (trunk.py:419-420).
* ``piquet_embedding_fp32.npz`` -- the field table (cardgym/games/piquet/tokens.py
  FIELD_VOCAB, NUM_FIELDS, CARD_VOCAB; cards.py CARD_RANKS) and ``PiquetEmbedding.forward``
  (cardgym/games/piquet/model.py:318-341) in fp32 on the CPU (its ``embedding_bag`` path,
  model.py:248-250) at the reference actor's default shape.

Inputs and weights come from ``seeded.py`` (pure functions of a seed); each file stores
the SHA-256 of the inputs it was made from, which the tests check first.
"""

from __future__ import annotations

import argparse
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))

import seeded  # noqa: E402
from cases import (  # noqa: E402
    CHUNK,
    PIQUET,
    STEP1,
    TRUNK,
    piquet_tokens,
    pool_contents,
    trunk_inputs,
    write_positions,
)


def _trunk_case(reference_modules, case, weights, out: dict) -> None:
    KVCache = reference_modules["KVCache"]
    trunk = reference_modules["trunk"]
    inputs = trunk_inputs(case)
    pool_k, pool_v = pool_contents(case)
    cache = KVCache(
        n_layers=TRUNK["n_layers"], kv_heads=TRUNK["n_kv_heads"], head_dim=TRUNK["d_model"] // TRUNK["n_heads"],
        capacity=case["capacity"], max_len=case["max_len"], device="cpu", dtype=torch.bfloat16,
    )
    for layer in range(TRUNK["n_layers"]):
        cache.k[layer].copy_(torch.from_numpy(pool_k[layer]).to(torch.bfloat16))
        cache.v[layer].copy_(torch.from_numpy(pool_v[layer]).to(torch.bfloat16))
    with torch.no_grad():
        x, ple, values = trunk.condition(torch.from_numpy(inputs["x"]), None, None)
        hidden = trunk.forward_ragged(
            x, ple, values, cache, torch.from_numpy(inputs["positions"]), torch.from_numpy(inputs["readout"]),
            span=None, rows=torch.from_numpy(inputs["rows"]),
        )
    name = case["name"]
    out[f"{name}_inputs_sha256"] = np.array(seeded.digest({**inputs, "pool_k": pool_k, "pool_v": pool_v}))
    out[f"{name}_hidden"] = hidden.numpy().astype(np.float32)
    # The slots the step wrote, [layers, B, T, kv_heads, head_dim] as bf16 bit patterns; the
    # tests check every other slot against the pool before the step.
    wp = torch.from_numpy(write_positions(case, inputs["positions"]))
    rows = torch.from_numpy(inputs["rows"])[:, None].expand_as(wp)
    for side, pool in (("k", cache.k), ("v", cache.v)):
        written = torch.stack([pool[l][rows, :, wp] for l in range(TRUNK["n_layers"])])
        out[f"{name}_{side}_written"] = written.view(torch.int16).numpy()
    # Unwritten slots are unchanged in the reference too (checked here, once).
    for layer in range(TRUNK["n_layers"]):
        for side, pool, before in (("k", cache.k, pool_k), ("v", cache.v, pool_v)):
            after = pool[layer].float().numpy().copy()
            after[rows.numpy(), :, wp.numpy()] = before[layer][rows.numpy(), :, wp.numpy()]
            assert np.array_equal(after, before[layer]), f"{name}: the reference changed an unwritten slot"


def make_trunk(reference_modules, out_dir: Path) -> Path:
    Trunk, TrunkConfig = reference_modules["Trunk"], reference_modules["TrunkConfig"]
    config = TrunkConfig(**{k: TRUNK[k] for k in ("d_model", "n_layers", "n_heads", "n_kv_heads", "d_ff")})
    torch.manual_seed(0)
    trunk = Trunk(config).eval()
    shapes = {k: tuple(v.shape) for k, v in trunk.state_dict().items()}
    weights = seeded.state_values(shapes, TRUNK["seed"])
    trunk.load_state_dict({k: torch.from_numpy(v) for k, v in weights.items()})
    out = {"weights_sha256": np.array(seeded.digest(weights))}
    reference_modules = {**reference_modules, "trunk": trunk}
    for case in (STEP1, CHUNK):
        _trunk_case(reference_modules, case, weights, out)
    path = out_dir / "trunk_ragged_bf16kv.npz"
    np.savez_compressed(path, **out)
    return path


def make_piquet(out_dir: Path) -> Path:
    from cardgym.games.piquet import cards as ref_cards
    from cardgym.games.piquet import tokens as ref_tokens
    from cardgym.games.piquet.model import PiquetEmbedding, PiquetModelConfig

    config = PiquetModelConfig()
    torch.manual_seed(0)
    embedding = PiquetEmbedding(config, PIQUET["ple_width"], PIQUET["value_width"]).eval()
    shapes = {k: tuple(v.shape) for k, v in embedding.state_dict().items()}
    weights = seeded.state_values(shapes, PIQUET["seed"])
    embedding.load_state_dict({k: torch.from_numpy(v) for k, v in weights.items()})
    tokens = piquet_tokens(tuple(ref_tokens.FIELD_VOCAB))
    with torch.no_grad():
        x, ple, values = embedding(torch.from_numpy(tokens))
        cards = embedding.kept
    out = {
        "field_vocab": np.asarray(ref_tokens.FIELD_VOCAB, dtype=np.int64),
        "num_fields": np.array(ref_tokens.NUM_FIELDS),
        "card_start": np.array(ref_tokens.CARD_START),
        "card_vocab": np.array(ref_tokens.CARD_VOCAB),
        "card_ranks": np.asarray(ref_cards.CARD_RANKS, dtype=np.int64),
        "offsets": embedding.offsets.numpy().astype(np.int64),
        "config": np.array([config.d_model, config.card_width, config.card_hidden, config.card_layers,
                            config.card_kernel, PIQUET["ple_width"], PIQUET["value_width"]], dtype=np.int64),
        "state_names": np.array(sorted(shapes)),
        "weights_sha256": np.array(seeded.digest(weights)),
        "tokens": tokens,
        "x": x.numpy().astype(np.float32),
        "ple": ple.numpy().astype(np.float32),
        "values": values.numpy().astype(np.float32),
        "cards": cards.numpy().astype(np.float32),
    }
    path = out_dir / "piquet_embedding_fp32.npz"
    np.savez_compressed(path, **out)
    return path


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--reference", default="/root/reference")
    parser.add_argument("--out", default=str(HERE))
    args = parser.parse_args()
    sys.path.insert(0, args.reference)
    from cardgym.nn.kv_cache import KVCache
    from cardgym.nn.trunk import Trunk, TrunkConfig

    torch.set_num_threads(8)
    out_dir = Path(args.out)
    modules = {"KVCache": KVCache, "Trunk": Trunk, "TrunkConfig": TrunkConfig}
    for path in (make_trunk(modules, out_dir), make_piquet(out_dir)):
        print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
