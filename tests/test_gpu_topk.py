"""Bounded top-k on the GPU vs the stable-sort oracle (bit-exact values and indices)."""

import pytest
import torch

from oracle.topk import topk as oracle_topk

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def run(logits, k, block_size=None):

    from sonic_sampler.interface import UnshardedBoundedTopK

    topk = UnshardedBoundedTopK.initialize(vocab_size=logits.size(-1), batch_size=logits.size(0),
                                           k=k, block_size=block_size, device=DEV)
    values, indices = topk(logits.to(DEV))
    torch.cuda.synchronize()

    return values.cpu(), indices.cpu()


def check(logits, k, block_size=None):

    values, indices = run(logits, k, block_size)
    ev, ei = oracle_topk(logits, k)

    assert torch.equal(indices, ei), (indices[:2, :8], ei[:2, :8])
    assert torch.equal(values.view(torch.int16 if values.dtype == torch.bfloat16 else torch.int32),
                       ev.view(torch.int16 if ev.dtype == torch.bfloat16 else torch.int32))


def test_config0_fp32_k32():

    from bench import c0_inputs

    logits, k = c0_inputs()
    print("config 0: B=8 V=32000 fp32 k=32", flush=True)
    check(logits, k)


@pytest.mark.parametrize("k", [1, 2, 32, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_ties_and_k(k, dtype):

    g = torch.Generator().manual_seed(k)
    # heavy ties: few distinct values
    logits = torch.randint(-4, 5, (6, 8192), generator=g).to(dtype)
    print(f"ties k={k} {dtype}", flush=True)
    check(logits, k, block_size=1024)


@pytest.mark.parametrize("vocab,block", [(128256, None), (151936, None), (262144, None), (5000, 1024), (40003, 2048),
                                         (131072, 16384), (40004, 16384)])
def test_bf16_shapes(vocab, block):

    from bench import spiked_logits

    logits = spiked_logits(4, vocab, seed=vocab)
    print(f"bf16 V={vocab} block={block}", flush=True)
    check(logits, 128, block)


def test_signed_zeros_and_infinities():

    x = torch.zeros(2, 4096)
    x[0, ::3] = -0.0
    x[1, :100] = float("-inf")
    x[1, 200:260] = float("inf")
    x[:, 1000:1010] = torch.arange(10, dtype=torch.float32)

    for dtype in (torch.float32, torch.bfloat16):

        print(f"zeros/inf {dtype}", flush=True)
        values, indices = run(x.to(dtype), 128, 1024)
        ev, ei = oracle_topk(x.to(dtype), 128)
        assert torch.equal(indices, ei)
        assert torch.equal(values.float().abs(), ev.float().abs())


@pytest.mark.parametrize("vocab,k,dtype", [
    (32000, 1, torch.float32), (32000, 128, torch.float32), (30001, 64, torch.float32),
    (32768, 16, torch.bfloat16), (20001, 128, torch.bfloat16), (1500, 8, torch.float32)])
def test_one_launch_rows(vocab, k, dtype):
    """64 rows under the automatic layout choice, several k, a vocabulary that is not a multiple of
    4 (per-element loads). The cases with 16385-32768 columns at k <= 32 (k = 1 at 32000, k = 16 at
    32768) take the one-workgroup-per-row kernel; the other four take the tile grid (k > 32, or
    at most 16384 columns)."""

    from bench import spiked_logits

    logits = spiked_logits(64, vocab, seed=vocab + k, dtype=dtype)
    print(f"one-launch rows V={vocab} k={k} {dtype}", flush=True)
    check(logits, k, 1024)


def test_one_launch_rows_concentrated_values():
    """One wave holding more than 128 values at or above the bound takes the exact selection."""

    g = torch.Generator().manual_seed(3)
    logits = torch.randn(4, 32000, generator=g)
    logits[:, 4 * 64 * 3:4 * 64 * 3 + 600] = 50.0 + torch.rand(4, 600, generator=g)   # wave 0's columns
    print("one-launch rows, concentrated", flush=True)
    check(logits, 128, 1024)


@pytest.mark.parametrize("vocab,k,dtype", [(32000, 32, torch.float32), (30001, 128, torch.bfloat16),
                                           (8192, 8, torch.float32), (32768, 1, torch.bfloat16),
                                           (16385, 2, torch.float32)])
def test_one_workgroup_per_row_strategy(vocab, k, dtype):
    """ss_topk with strategy ROWWISE (one launch, one 1024-thread workgroup per row), called
    through the C-ABI: bit-exact against the oracle, including rows whose survivors need two sorting
    waves, overflow the survivor list, or tie heavily (the exact selection)."""

    import ctypes

    from bench import spiked_logits
    from sonic_sampler import _native

    rows = 8
    g = torch.Generator().manual_seed(1)
    logits = spiked_logits(rows, vocab, seed=vocab, dtype=dtype)
    logits[1] = torch.randint(-3, 4, (vocab,), generator=g).to(dtype)
    # 200 and 600 raised values spread over every wave's columns: more survivors than one sorted
    # wave holds (two waves sort them), and more than the survivor list holds (exact selection)
    for r, n in ((2, 200), (3, 600)):
        cols = torch.randperm(vocab, generator=g)[:n]
        logits[r, cols] = (30.0 + 10.0 * torch.rand(n, generator=g)).to(dtype)
    x = logits.to(DEV)
    values = torch.empty(rows, k, dtype=dtype, device=DEV)
    indices = torch.empty(rows, k, dtype=torch.int32, device=DEV)
    scratch = torch.empty(rows, 64 * k, dtype=torch.int64, device=DEV)   # not used by this layout
    args = _native.TopKArgs(
        logits=x.data_ptr(), stride_logits=x.stride(0),
        dtype=_native.SS_DTYPE_F32 if dtype == torch.float32 else _native.SS_DTYPE_BF16,
        rows=rows, vocab_size=vocab, k=k, block_n=1024, strategy=_native.STRATEGY_ROWWISE,
        scratch=scratch.data_ptr(), stride_scratch=scratch.stride(0) * (2 if dtype == torch.float32 else 4),
        values=values.data_ptr(), indices=indices.data_ptr(), stream=_native.stream_of(x))
    print(f"ss_topk rowwise V={vocab} k={k} {dtype}", flush=True)
    _native.check(_native.load().ss_topk(ctypes.byref(args)), "ss_topk")
    torch.cuda.synchronize()
    ev, ei = oracle_topk(logits, k)
    assert torch.equal(indices.cpu(), ei)
    assert torch.equal(values.cpu().float(), ev.float())


@pytest.mark.parametrize("k", [32, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_merge_paths_at_128_tiles(k, dtype):
    """V = 131072 at block 1024: 128 sorted lists of k candidates, of which the merge samples 4
    each. Rows whose top-k crowds into a few lists (merged whole), into more than 16 lists or ties
    everywhere (radix merge), and plain rows (sampled merge) must all be exact."""

    from bench import spiked_logits

    rows, vocab, block = 10, 131072, 1024
    g = torch.Generator().manual_seed(k)
    logits = spiked_logits(rows, vocab, seed=900 + k, dtype=torch.float32)

    for r in range(rows):

        kind = r % 5

        if kind == 3:

            logits[r] = torch.randint(-2, 2, (vocab,), generator=g).float()
            continue

        hot, per = {1: (3, k // 2), 2: (24, k // 4), 4: (12, k // 4)}.get(kind, (0, 0))

        for t in torch.randperm(vocab // block, generator=g)[:hot].tolist():

            cols = t * block + torch.randperm(block, generator=g)[:per]
            logits[r, cols] = 40.0 + torch.rand(per, generator=g) * 8.0

    print(f"top-k merge paths at 128 tiles: k={k} {dtype}", flush=True)
    check(logits.to(dtype), k, block)


@pytest.mark.parametrize("rows", [48, 160])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_many_narrow_rows_take_one_launch(dtype, rows):
    """48 and 160 rows of 32000 columns at k = 32 through the interface: the library's automatic
    choice is one 1024-thread workgroup per row; bit-exact against the oracle, with tied and
    crowded rows among them."""

    from bench import spiked_logits

    vocab, k = 32000, 32
    g = torch.Generator().manual_seed(11)
    logits = spiked_logits(rows, vocab, seed=12, dtype=torch.float32)
    logits[5] = torch.randint(-3, 4, (vocab,), generator=g).float()
    logits[6] = 0.5
    cols = torch.randperm(vocab, generator=g)[:300]
    logits[7, cols] = 30.0 + 10.0 * torch.rand(300, generator=g)
    logits = logits.to(dtype)
    print(f"many narrow rows, one launch: {rows} rows {dtype}", flush=True)
    check(logits, k, 1024)


@pytest.mark.parametrize("rows", [8, 64])
def test_graph_replay(rows):
    """ss_topk captured in a hipGraph (8 rows: tile and merge launches; 64 rows: one workgroup per
    row) and replayed over new logits copied into the captured input: every replay equals the
    eager call and the oracle."""

    from bench import spiked_logits
    from sonic_sampler.interface import UnshardedBoundedTopK

    vocab, k = 32000, 32
    sets = [spiked_logits(rows, vocab, seed=500 + i, dtype=torch.float32) for i in range(3)]
    x = sets[0].to(DEV)
    topk = UnshardedBoundedTopK.initialize(vocab_size=vocab, batch_size=rows, k=k, device=DEV)
    eager = []

    for s in sets:

        x.copy_(s)
        values, indices = topk(x)
        eager.append((values.clone(), indices.clone()))

    torch.cuda.synchronize()
    print(f"top-k graph replay: {rows} rows; capturing", flush=True)
    x.copy_(sets[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    with torch.cuda.stream(side):

        topk(x)

    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()

    with torch.cuda.graph(graph):

        captured = topk(x)

    for rnd, i in enumerate([1, 2, 0, 2, 1]):

        x.copy_(sets[i])
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"replay {rnd}: input set {i}", flush=True)
        assert torch.equal(captured[0], eager[i][0]) and torch.equal(captured[1], eager[i][1])

        if rnd < 3:

            ev, ei = oracle_topk(sets[i], k)
            assert torch.equal(captured[1].cpu(), ei)
            assert torch.equal(captured[0].cpu().view(torch.int32), ev.view(torch.int32))


@pytest.mark.parametrize("k", [32, 128])
def test_more_than_512_tiles(k):
    """586 tiles of 1024 columns: the merge takes the per-row radix merge over every candidate."""

    from bench import spiked_logits

    logits = spiked_logits(3, 600_000, seed=600 + k)
    print(f"top-k over 586 tiles, k={k}", flush=True)
    check(logits, k, block_size=1024)
