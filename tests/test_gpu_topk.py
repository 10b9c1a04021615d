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


@pytest.mark.parametrize("vocab,block", [(128256, None), (151936, None), (262144, None), (5000, 1024), (40003, 2048)])
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
