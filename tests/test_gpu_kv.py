"""KV pool kernels against the oracle's restatement of cardgym/nn/kv_cache.py: bit-exact.

Cache contents are compared as raw bit patterns (NaN only as NaN: torch's own NaN payloads
differ between its cast paths), on inputs that contain the values where a cast can go
wrong: exact rounding ties, NaN, +-inf, -0.0, subnormals and values that overflow fp16.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from card_playing_gym_amd.nn.kv_cache import KVCache
from oracle.reference_path import RefCache

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def bits(t: torch.Tensor) -> torch.Tensor:
    t = t.detach().cpu().contiguous()
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)


def tricky(shape, gen) -> torch.Tensor:
    """fp32 values with every cast edge case mixed into normal draws."""

    x = torch.randn(shape, generator=gen)
    flat = x.view(-1)
    specials = torch.tensor(
        [float("nan"), float("inf"), float("-inf"), -0.0, 0.0, 1e-40, -3e-39, 65520.0, 70000.0, 6e-8, 3e-8, 1.0 + 2**-8,
         1.0 + 3 * 2**-8, -(1.0 + 2**-8), 2**-126, 5.9604645e-08]
    )
    # Exact bf16 ties: low 16 bits = 0x8000 on both even and odd kept mantissas.
    ties = torch.from_numpy(np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x40498000], dtype=np.uint32).view(np.float32))
    edge = torch.cat([specials, ties])
    idx = torch.randperm(flat.numel(), generator=gen)[: edge.numel()]
    flat[idx] = edge
    return x


def make_pair(dtype, device, capacity=9, max_len=17, n_layers=2, kv_heads=2, head_dim=32):
    native = KVCache(n_layers=n_layers, kv_heads=kv_heads, head_dim=head_dim, capacity=capacity, max_len=max_len,
                     device=device, dtype=dtype)
    ref = RefCache(n_layers, kv_heads, head_dim, capacity, max_len, dtype)
    return native, ref


def assert_bits_equal(got: torch.Tensor, want: torch.Tensor, what: str) -> None:
    """Exact bit equality, except that NaN payloads only need to be NaN on both sides:
    torch itself writes different NaN patterns on different paths (its scalar bf16 cast
    gives 0x7FC0, its vectorised CPU cast 0xFFFF)."""

    got, want = got.detach().cpu(), want.detach().cpu()
    nan_g, nan_w = torch.isnan(got.float()), torch.isnan(want.float())
    assert torch.equal(nan_g, nan_w), f"{what}: NaN positions differ"
    same = (bits(got) == bits(want)) | nan_g
    if not bool(same.all()):
        idx = (~same).nonzero()[:5]
        detail = [(tuple(i.tolist()), float(got[tuple(i)]), float(want[tuple(i)]), int(bits(got)[tuple(i)]),
                   int(bits(want)[tuple(i)])) for i in idx]
        raise AssertionError(f"{what}: {int((~same).sum())} elements differ, first {detail}")


def assert_same(native: KVCache, ref: RefCache):
    for layer in range(ref.n_layers):
        assert_bits_equal(native.k[layer], ref.k[layer], f"k layer {layer}")
        assert_bits_equal(native.v[layer], ref.v[layer], f"v layer {layer}")


@pytest.mark.parametrize("cache_dtype", DTYPES)
@pytest.mark.parametrize("src_dtype", DTYPES)
def test_write_step_is_bit_exact(device, cache_dtype, src_dtype):
    gen = torch.Generator().manual_seed(1)
    native, ref = make_pair(cache_dtype, device)
    B, T, KVH, D = 6, 3, 2, 32
    rows = torch.randperm(9, generator=gen)[:B]
    starts = torch.randint(0, 17 - T, (B,), generator=gen)
    positions = starts[:, None] + torch.arange(T)[None, :]
    # [B, T, KVH, D] transposed to [B, KVH, T, D]: the strided view the QKV split hands over.
    k = tricky((B, T, KVH, D), gen).to(src_dtype).transpose(1, 2)
    v = tricky((B, T, KVH, D), gen).to(src_dtype).transpose(1, 2)
    for layer in range(2):
        native.write_step(layer, rows.to(device), positions.to(device), k.to(device), v.to(device))
        ref.write_step(layer, rows, positions, k, v)
    torch.cuda.synchronize()
    assert_same(native, ref)


@pytest.mark.parametrize("cache_dtype", DTYPES)
def test_write_step_single_position_form(device, cache_dtype):
    gen = torch.Generator().manual_seed(2)
    native, ref = make_pair(cache_dtype, device)
    B = 9
    rows = torch.randperm(9, generator=gen)
    positions = torch.randint(0, 17, (B,), generator=gen)
    k = tricky((B, 2, 1, 32), gen)
    v = tricky((B, 2, 1, 32), gen)
    native.write_step(1, rows.to(device), positions.to(device), k.to(device), v.to(device))
    ref.write_step(1, rows, positions, k, v)
    torch.cuda.synchronize()
    assert_same(native, ref)


@pytest.mark.parametrize("cache_dtype", DTYPES)
@pytest.mark.parametrize("dense", [True, False])
def test_write_range_is_bit_exact(device, cache_dtype, dense):
    gen = torch.Generator().manual_seed(3)
    native, ref = make_pair(cache_dtype, device)
    B, T = 5, 7
    rows = None if dense else torch.randperm(9, generator=gen)[:B]
    k = tricky((B, 2, T, 32), gen)
    v = tricky((B, 2, T, 32), gen)
    native.write_range(0, None if rows is None else rows.to(device), 4, k.to(device), v.to(device))
    ref.write_range(0, rows, 4, k, v)
    torch.cuda.synchronize()
    assert_same(native, ref)


@pytest.mark.parametrize("cache_dtype", DTYPES)
def test_gathered_read_matches(device, cache_dtype):
    gen = torch.Generator().manual_seed(4)
    native, ref = make_pair(cache_dtype, device)
    fill_k = tricky((9, 2, 17, 32), gen).to(cache_dtype)
    fill_v = tricky((9, 2, 17, 32), gen).to(cache_dtype)
    native.k[1].copy_(fill_k.to(device))
    native.v[1].copy_(fill_v.to(device))
    ref.k[1].copy_(fill_k)
    ref.v[1].copy_(fill_v)
    rows = torch.tensor([3, 3, 0, 8, 5])
    k, v = native.read(1, rows.to(device), 11)
    rk, rv = ref.read(1, rows, 11)
    assert_bits_equal(k, rk, 'k')
    assert_bits_equal(v, rv, 'v')
    dk, dv = native.read(1, None, 6, count=4)
    assert dk.data_ptr() == native.k[1].data_ptr()  # zero-copy prefix view
    assert dk.shape == (4, 2, 6, 32) and dv.shape == (4, 2, 6, 32)


def test_copy_rows_moves_prefixes(device):
    """tests/nn/test_trunk.py:81-88 of the reference, on the device pool."""

    cache = KVCache(n_layers=2, kv_heads=1, head_dim=2, capacity=4, max_len=5, device=device)
    for layer in range(2):
        cache.k[layer][:] = torch.arange(4, dtype=torch.float32, device=device).view(4, 1, 1, 1)
        cache.v[layer][:] = -torch.arange(4, dtype=torch.float32, device=device).view(4, 1, 1, 1)
    cache.copy_rows(torch.tensor([2, 3]), torch.tensor([1, 2]), length=3)
    assert cache.k[1][:, 0, 0, 0].tolist() == [0.0, 2.0, 3.0, 3.0]
    assert cache.v[0][1, 0, 3, 0].item() == -1.0  # beyond the copied length


@pytest.mark.parametrize("cache_dtype", DTYPES)
def test_copy_rows_random_overlap(device, cache_dtype):
    gen = torch.Generator().manual_seed(5)
    native, ref = make_pair(cache_dtype, device)
    for layer in range(2):
        fk = tricky((9, 2, 17, 32), gen).to(cache_dtype)
        fv = tricky((9, 2, 17, 32), gen).to(cache_dtype)
        native.k[layer].copy_(fk.to(device))
        native.v[layer].copy_(fv.to(device))
        ref.k[layer].copy_(fk)
        ref.v[layer].copy_(fv)
    sources = torch.tensor([2, 4, 5, 8])
    targets = torch.tensor([1, 2, 4, 5])
    native.copy_rows(sources, targets, 13)
    ref.copy_rows(sources, targets, 13)
    torch.cuda.synchronize()
    assert_same(native, ref)


def test_out_of_range_indices_are_skipped_and_reported(device, monkeypatch):
    native, _ = make_pair(torch.float32, device)
    k = torch.ones((2, 2, 1, 32), device=device)
    expected = native.k[0].clone()
    expected[1, :, 3] = 1.0
    # Row 99 does not exist: the kernel skips it (no fault), the in-range row is written.
    native.write_step(0, torch.tensor([99, 1]), torch.tensor([3, 3]), k, k)
    torch.cuda.synchronize()
    assert torch.equal(native.k[0], expected)
    monkeypatch.setenv("CARDGYM_HIP_CHECK", "1")
    with pytest.raises(IndexError):
        native.write_step(0, torch.tensor([99, 1]), torch.tensor([3, 3]), k, k)
    with pytest.raises(IndexError):
        native.write_step(0, torch.tensor([0, 1]), torch.tensor([3, 17]), k, k)


def fill_pair(native, ref, gen):
    for layer in range(native.n_layers):
        shape = tuple(native.k[layer].shape)
        fk = tricky(shape, gen).to(native.dtype)
        fv = tricky(shape, gen).to(native.dtype)
        native.k[layer].copy_(fk.to(native.device))
        native.v[layer].copy_(fv.to(native.device))
        ref.k[layer].copy_(fk)
        ref.v[layer].copy_(fv)


@pytest.mark.parametrize("cache_dtype", DTYPES)
@pytest.mark.parametrize(
    "sources,targets",
    [
        ([1, 2], [2, 1]),  # swap: both rows must see the other's old contents
        ([5, 0, 7, 3], [2, 8, 6, 1]),  # disjoint: the direct path
        ([3, 3, 3], [4, 5, 6]),  # one source fanned out
        ([0, 1, 2, 3, 4, 5, 6, 7], [1, 2, 3, 4, 5, 6, 7, 8]),  # shift up by one: a chain of overlaps
        ([1, 5, 6, 4], [2, 1, 7, 4]),  # staged (1), direct (5, 6) and a row onto itself (4) in one call
    ],
)
def test_copy_rows_overlap_patterns(device, cache_dtype, sources, targets):
    gen = torch.Generator().manual_seed(11)
    native, ref = make_pair(cache_dtype, device)
    fill_pair(native, ref, gen)
    native.copy_rows(torch.tensor(sources), torch.tensor(targets), 17)
    ref.copy_rows(torch.tensor(sources), torch.tensor(targets), 17)
    torch.cuda.synchronize()
    assert_same(native, ref)


@pytest.mark.parametrize("stacked", [True, False])
def test_copy_rows_chunked_compaction(device, stacked):
    """selfplay.py:353-372's compaction pattern (survivors moved down, seats kept in order)
    with a chunk cap small enough that the copy runs in many chunks, so overlaps cross
    chunk boundaries exactly as the reference orders them."""

    gen = torch.Generator().manual_seed(12)
    native, ref = make_pair(torch.bfloat16, device, capacity=300, max_len=24, n_layers=3)
    fill_pair(native, ref, gen)
    for cache in (native, ref):
        cache.COPY_CHUNK_BYTES = 7 * 2 * 19 * 32 * 2 * (3 if stacked else 1)
        cache.stacked = stacked
    alive = torch.rand(100, generator=gen) < 0.6
    seats = 3
    survivors = torch.nonzero(alive).flatten()
    sources = (survivors[:, None] * seats + torch.arange(seats)).flatten()
    targets = torch.arange(sources.numel())
    native.copy_rows(sources, targets, 19)
    ref.copy_rows(sources, targets, 19)
    torch.cuda.synchronize()
    assert_same(native, ref)


@pytest.mark.parametrize("cache_dtype,head_dim", [(torch.bfloat16, 3), (torch.float16, 6), (torch.float32, 2), (torch.float32, 5)])
def test_copy_rows_narrow_positions(device, cache_dtype, head_dim):
    """Position widths that are not a multiple of 16 bytes (2-, 4- and 8-byte accesses)."""

    gen = torch.Generator().manual_seed(13)
    native, ref = make_pair(cache_dtype, device, head_dim=head_dim)
    fill_pair(native, ref, gen)
    sources, targets = torch.tensor([4, 5, 0]), torch.tensor([5, 3, 4])
    native.copy_rows(sources, targets, 9)
    ref.copy_rows(sources, targets, 9)
    torch.cuda.synchronize()
    assert_same(native, ref)


def test_copy_rows_workspace_is_checked(device):
    from card_playing_gym_amd import _native as nat

    native, _ = make_pair(torch.float32, device)
    layers = native.layer_array()
    src = torch.tensor([1], device=device)
    dst = torch.tensor([2], device=device)
    need = nat.lib().cg_kv_copy_workspace_size(layers, 2, 1, 5)
    assert need == 256 + 2 * 2 * 5 * 32 * 4  # classification, then one layer's K and V prefixes
    small = torch.empty(need - 16, dtype=torch.uint8, device=device)
    with pytest.raises(ValueError, match="workspace too small"):
        nat.call("cg_kv_copy_rows_layers", layers, 2, src.data_ptr(), dst.data_ptr(), 1, 5, nat.CG_COPY_AUTO,
                 small.data_ptr(), small.numel(), native._stream())


def ordered(sources, targets) -> bool:
    """No pair writes a row that a later pair reads (the chunks the ordered walk takes)."""

    last = {}
    for k, s in enumerate(sources):
        last[s] = k
    return all(last.get(t, -1) <= i for i, t in enumerate(targets))


# Large enough (8 layers x 2 heads x K/V x 2048 16-byte slices) for the per-slice ordered
# walk; smaller copies always take the staged path.
WALK = dict(capacity=48, max_len=520, n_layers=8, kv_heads=2, head_dim=32)


@pytest.mark.parametrize(
    "sources,targets,is_ordered",
    [
        ([6, 7, 8, 9, 13, 14, 15, 16, 17, 30, 31], [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10], True),  # compaction
        ([20, 21, 22], [30, 31, 32], True),  # disjoint
        ([3, 3, 3], [4, 5, 6], True),  # fan-out
        ([1, 5, 6, 4], [2, 1, 7, 4], True),  # a row onto itself, and a write after its read
        ([1, 2], [2, 1], False),  # swap
        (list(range(12)), list(range(1, 13)), False),  # shift up: each write precedes its read
    ],
)
@pytest.mark.parametrize("indices_on", ["host", "device"])
def test_copy_rows_ordered_walk(device, sources, targets, is_ordered, indices_on):
    """Host indices are classified on the host (the walk alone runs for ordered chunks);
    device indices on the device."""

    assert ordered(sources, targets) == is_ordered
    gen = torch.Generator().manual_seed(14)
    native, ref = make_pair(torch.bfloat16, device, **WALK)
    fill_pair(native, ref, gen)
    where = "cpu" if indices_on == "host" else device
    native.copy_rows(torch.tensor(sources, device=where), torch.tensor(targets, device=where), 512)
    ref.copy_rows(torch.tensor(sources), torch.tensor(targets), 512)
    torch.cuda.synchronize()
    assert_same(native, ref)


@pytest.mark.parametrize("stacked", [True, False])
@pytest.mark.parametrize("indices_on", ["host", "device"])
def test_copy_rows_ordered_walk_in_chunks(device, stacked, indices_on):
    gen = torch.Generator().manual_seed(15)
    native, ref = make_pair(torch.float16, device, **WALK)
    fill_pair(native, ref, gen)
    for cache in (native, ref):
        cache.COPY_CHUNK_BYTES = 5 * 2 * 512 * 32 * 2 * (8 if stacked else 1)  # five rows a chunk
        cache.stacked = stacked
    alive = torch.tensor([0, 1, 1, 0, 1, 0, 0, 1, 1, 1, 0, 1, 1, 0, 1, 1], dtype=torch.bool)
    survivors = torch.nonzero(alive).flatten()
    sources = (survivors[:, None] * 3 + torch.arange(3)).flatten()
    targets = torch.arange(sources.numel())
    moved = sources != targets
    where = "cpu" if indices_on == "host" else device
    native.copy_rows(sources[moved].to(where), targets[moved].to(where), 512)
    ref.copy_rows(sources[moved], targets[moved], 512)
    torch.cuda.synchronize()
    assert_same(native, ref)
