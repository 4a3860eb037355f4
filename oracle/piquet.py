"""ORACLE -- test infrastructure only.

A CPU restatement, in eager PyTorch, of Piquet's token embedder: the per-field lookups and
the card grid that turn a [..., 64] token (32 fields, 32 card codes) into the trunk's input
sum, its per-layer and value embeddings, and the per-card features the card heads read.
It is the checker for the HIP embedder and the "reference path" timed beside it; it is
never part of the product.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
baseline leg may import it.

What it restates (paths into maxrlinder/card_playing_gym):
  * constants           cardgym/games/piquet/tokens.py:108-152 (fields, vocabularies),
                        cardgym/games/piquet/cards.py:11-14, 26-35, 78 (card = suit * 8 +
                        rank), cardgym/games/piquet/engine.py:50-56 (hand, talon, heads)
  * ``grid_norm``       cardgym/games/piquet/model.py:114-125 (GridNorm)
  * ``grid_block``      cardgym/games/piquet/model.py:128-177 (GridBlock: block-Toeplitz
                        rank convolution, zero-padded; suit pooling; across projection)
  * ``cards``           cardgym/games/piquet/model.py:234-241 (CardGrid.cards, unfused)
  * ``summary``         cardgym/games/piquet/model.py:243-245
  * ``field_sums``      cardgym/games/piquet/model.py:255-270 (the one-hot GEMM of the
                        CUDA path) and 248-250 (embedding_bag, the CPU path)
  * ``forward``         cardgym/games/piquet/model.py:318-341 (PiquetEmbedding.forward)

Precision modes, as in oracle/reference_path.py: ``"fp32"`` (no autocast) and ``"bf16"``
(the rounding points of torch.autocast("cuda", bfloat16), written as explicit casts):
embeddings and norms in fp32; every nn.Linear, F.linear and ``@`` takes bf16 operands and
returns bf16 (the Toeplitz einsum of bf16 weights is exact); GELU runs on its bf16 input;
additions of two bf16 tensors round to bf16; bf16 + fp32 promotes to fp32.

Parity status: pinned by tests/test_oracle.py -- the convolution against
``torch.nn.functional.conv1d`` with zero padding, the one-hot sums against
``embedding_bag``, the norm against its closed form, suit pooling against the mean, and
the whole grid's equivariance under suit permutations (the model's stated symmetry).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

NUM_SUITS, NUM_RANKS = 4, 8
NUM_CARDS = NUM_SUITS * NUM_RANKS
NUM_FIELDS = 32
CARD_START = NUM_FIELDS
CARD_VOCAB = 12
_HEADS, _TRICKS, _TALON = 3, 12, 8
_TOTAL_VOCAB = 120 + 21
_LEAD_VOCAB = 2 * (60 + 14) + 1
FIELD_VOCAB = (
    8, 1 + _HEADS, 3, 2, NUM_CARDS + 1, 9, 9, 4, 4, 9, 76, 9, 3, 4, 64, 5, 3,
    _TRICKS + 1, 3, 5, _TRICKS + 1, _TRICKS + 1, 100, 100, _TOTAL_VOCAB, _TOTAL_VOCAB,
    6, 2, _TALON + 1, 16, 4, _LEAD_VOCAB,
)
FIELD_OFFSETS = tuple(sum(FIELD_VOCAB[:i]) for i in range(NUM_FIELDS))
CARD_RANKS = tuple(card & 7 for card in range(NUM_CARDS))


class RefPiquetEmbedding:
    """PiquetEmbedding.forward over a reference-named state dict (``embedding.*``)."""

    def __init__(self, state: dict[str, torch.Tensor], card_layers: int, kernel: int, precision: str = "bf16",
                 prefix: str = "embedding.", eps: float = 1e-5):
        if precision not in ("fp32", "bf16"):
            raise ValueError(f"unknown precision {precision!r}")
        self.bf16 = precision == "bf16"
        self.s = {k[len(prefix):]: v for k, v in state.items() if k.startswith(prefix)}
        self.layers, self.kernel, self.eps = card_layers, kernel, eps
        self._consts: dict = {}  # per device: field offsets, card ranks (no copies under capture)

    def _const(self, device):
        if device not in self._consts:
            self._consts[device] = (torch.tensor(FIELD_OFFSETS, device=device), torch.tensor(CARD_RANKS, device=device))
        return self._consts[device]

    # -- precision policy ------------------------------------------------------

    def _b(self, t):
        return t.bfloat16() if self.bf16 else t

    def lin(self, x, weight, bias=None):
        return F.linear(self._b(x), self._b(weight), None if bias is None else self._b(bias))

    def mm(self, a, b):
        return self._b(a) @ self._b(b)

    def add(self, a, b):
        # bf16 + bf16 stays bf16 (rounded once); anything with fp32 promotes.
        return a + b

    # -- the grid (model.py:114-245) ------------------------------------------

    def grid_norm(self, x, weight):
        return F.rms_norm(x.float(), (x.shape[-1],), weight.float(), self.eps).to(x.dtype)

    def toeplitz(self, block: int) -> torch.Tensor:
        """[8 * width, 8 * hidden]: entry (i w, o h) = W[h, w, i - o + kernel // 2] when that
        tap exists (model.py:154-166; zero padding, no wrap)."""

        w = self.s[f"grid.blocks.{block}.along_rank.weight"]  # [hidden, width, kernel]
        hidden, width, kernel = w.shape
        key = ("shifts", kernel, w.device, w.dtype)
        if key not in self._consts:  # a registered buffer in the reference (model.py:141-148)
            half = kernel // 2
            shifts = torch.zeros(kernel, NUM_RANKS, NUM_RANKS, dtype=w.dtype)
            for tap in range(kernel):
                for rank in range(NUM_RANKS):
                    source = rank + tap - half
                    if 0 <= source < NUM_RANKS:
                        shifts[tap, source, rank] = 1.0
            self._consts[key] = shifts.to(w.device)
        shifts = self._consts[key]
        t = torch.einsum("kio,hwk->iwoh", self._b(shifts), self._b(w))
        return t.reshape(NUM_RANKS * width, NUM_RANKS * hidden)

    def along(self, block: int, rows):
        """Rank convolution of each suit row [N, suits, 8 * width] -> [N, suits, 8 * hidden]."""

        p = f"grid.blocks.{block}."
        return self.lin(rows, self.toeplitz(block).t(), self.s[p + "along_rank.bias"].repeat(NUM_RANKS))

    def pooled(self, rows):
        """Mean over suits [N, suits, 8 * width] -> [N, 8, width], as a [1, 4] matmul."""

        pool = torch.full((1, NUM_SUITS), 1.0 / NUM_SUITS, dtype=rows.dtype, device=rows.device)
        return self.mm(pool, rows).view(rows.shape[0], NUM_RANKS, -1)

    def grid_block(self, block: int, grid):  # [N, suits, ranks, width] fp32
        p = f"grid.blocks.{block}."
        count, _, _, width = grid.shape
        hidden = self.s[p + "out.weight"].shape[1]
        rows = self.grid_norm(grid, self.s[p + "norm.weight"]).reshape(count, NUM_SUITS, NUM_RANKS * width)
        along = self.along(block, rows)
        pooled = self.pooled(rows)
        across = self.lin(pooled, self.s[p + "across_suits.weight"]).view(count, 1, NUM_RANKS * hidden)
        spread = torch.ones(NUM_SUITS, 1, dtype=across.dtype, device=across.device)
        mixed = self.add(along, self.mm(spread, across))
        out = self.lin(F.gelu(mixed).view(count, NUM_SUITS, NUM_RANKS, hidden), self.s[p + "out.weight"],
                       self.s[p + "out.bias"])
        return grid + out

    def cards(self, codes):  # [..., 32] -> [..., 32, width] fp32
        lead = codes.shape[:-1]
        ranks = self._const(codes.device)[1]
        grid = F.embedding(codes.long(), self.s["grid.code.weight"]) + F.embedding(ranks, self.s["grid.rank.weight"])
        width = grid.shape[-1]
        grid = grid.reshape(-1, NUM_SUITS, NUM_RANKS, width)
        for block in range(self.layers):
            grid = self.grid_block(block, grid)
        return self.grid_norm(grid, self.s["grid.norm.weight"]).reshape(*lead, NUM_CARDS, width)

    def summary(self, cards):
        return self.lin(cards.flatten(-2), self.s["grid.summary.weight"])

    # -- field lookups (model.py:248-270) ---------------------------------------

    def tables(self):
        names = ["fields.weight"] + [n for n in ("ple_fields.weight", "value_fields.weight") if n in self.s]
        return [self.s[n] for n in names]

    def field_sums(self, ids):
        """The CUDA path's one-hot GEMM: [..., 32] ids (offsets added) -> one sum per table."""

        tables = self.tables()
        flat = ids.reshape(-1, ids.shape[-1])
        dtype = torch.bfloat16 if self.bf16 else tables[0].dtype
        hot = torch.zeros(flat.shape[0], tables[0].shape[0], dtype=dtype, device=flat.device).scatter_(1, flat, 1.0)
        widths = [t.shape[1] for t in tables]
        sums = hot @ torch.cat(tables, dim=1).to(dtype)
        return [part.view(*ids.shape[:-1], w) for part, w in zip(sums.split(widths, dim=1), widths)]

    def forward(self, tokens):
        """(x, ple lookup or None, value lookup or None, cards) for [..., 64] tokens."""

        tokens = tokens.long()
        ids = tokens[..., :NUM_FIELDS] + self._const(tokens.device)[0]
        cards = self.cards(tokens[..., CARD_START:])
        summary = self.summary(cards)
        sums = iter(self.field_sums(ids))
        x = self.add(next(sums), summary)
        ple = next(sums) if "ple_fields.weight" in self.s else None
        values = next(sums) if "value_fields.weight" in self.s else None
        return x, ple, values, cards


def random_state(d_model: int, ple_width: int, value_width: int, width: int = 32, hidden: int = 64,
                 layers: int = 2, kernel: int = 3, seed: int = 0, scale: float = 1.0) -> dict[str, torch.Tensor]:
    """Random parameters under the reference's names (``embedding.*``).  The reference
    zero-initialises the PLE / value tables; tests use random ones so that they are seen."""

    g = torch.Generator().manual_seed(seed)
    rows = sum(FIELD_VOCAB)

    def r(*shape, std=0.02):
        return torch.randn(*shape, generator=g) * std * scale

    s = {
        "embedding.fields.weight": r(rows, d_model),
        "embedding.grid.code.weight": r(CARD_VOCAB, width, std=1.0),
        "embedding.grid.rank.weight": r(NUM_RANKS, width, std=1.0),
        "embedding.grid.norm.weight": 1.0 + r(width, std=0.1),
        "embedding.grid.summary.weight": r(d_model, NUM_CARDS * width, std=0.05),
    }
    if ple_width:
        s["embedding.ple_fields.weight"] = r(rows, ple_width)
    if value_width:
        s["embedding.value_fields.weight"] = r(rows, value_width)
    for b in range(layers):
        p = f"embedding.grid.blocks.{b}."
        s[p + "norm.weight"] = 1.0 + r(width, std=0.1)
        s[p + "along_rank.weight"] = r(hidden, width, kernel, std=0.1)
        s[p + "along_rank.bias"] = r(hidden, std=0.1)
        s[p + "across_suits.weight"] = r(hidden, width, std=0.1)
        s[p + "out.weight"] = r(width, hidden, std=0.1)
        s[p + "out.bias"] = r(width, std=0.1)
    return s


def random_tokens(n: int, seed: int = 0) -> torch.Tensor:
    """[n, 64] int64 tokens: every field uniform over its vocabulary, card codes over 12."""

    g = torch.Generator().manual_seed(seed)
    fields = torch.stack([torch.randint(0, v, (n,), generator=g) for v in FIELD_VOCAB], dim=1)
    codes = torch.randint(0, CARD_VOCAB, (n, NUM_CARDS), generator=g)
    return torch.cat([fields, codes], dim=1)
