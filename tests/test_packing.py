"""The packed argument structs of the eager call path (CPU).

``fused_singular``, ``fused_multistep`` and ``UnshardedBoundedTopK`` hand the library their
argument structs as bytes packed positionally (``_native.Packer``) instead of ctypes structs built
by keyword. These tests
pin that path two ways: the packer's layout against ctypes' own for every argument struct, and the
bytes each driver packs against a struct built field by field by name from the same tensors, for
calls that set every field a caller can reach. The packed entry point is also called into the
library's argument validation, which must answer as it does for the ctypes struct.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from sonic_sampler import _native
from sonic_sampler.interface.functional import singular as fs

STRUCTS = [_native.TopKArgs, _native.SingularArgs, _native.MultistepArgs, _native.IndexedCopyArgs]


def named_struct(cls, fields, values):
    """cls(**kw) from flat (name, value) pairs, the nested Philox member rebuilt from its parts."""

    kw, philox = {}, {}

    for name, value in zip(fields, values):

        member = name.split("_", 1)[1] if name.startswith("philox_") else None

        if member in ("seed", "offset", "enabled"):

            philox[member] = value

        else:

            kw[name] = value

    if philox:

        kw["philox"] = _native.Philox(**philox)

    return cls(**kw)


@pytest.mark.parametrize("cls", STRUCTS, ids=lambda c: c.__name__)
def test_packer_layout_is_the_ctypes_layout(cls):

    packer = _native.Packer(cls)
    g = torch.Generator().manual_seed(len(packer.fields))
    values = [int(v) for v in torch.randint(1, 2 ** 31 - 1, (len(packer.fields),), generator=g)]

    assert len(set(packer.fields)) == len(packer.fields)
    assert packer.pack(*values) == bytes(named_struct(cls, packer.fields, values))


@pytest.mark.parametrize("cls", STRUCTS, ids=lambda c: c.__name__)
def test_packer_takes_every_field_type_to_its_limits(cls):
    """Each field at its type's extremes (and -1 for the signed ones) packs to the ctypes bytes."""

    packer = _native.Packer(cls)
    codes = [code for *_, code in _native._flat_layout(cls)]
    limits = {"i": (-2 ** 31, 2 ** 31 - 1, -1), "q": (-2 ** 63, 2 ** 63 - 1, -1),
              "I": (0, 2 ** 32 - 1, 1), "Q": (0, 2 ** 64 - 1, 1)}

    for pick in range(3):

        values = [limits[c][(pick + j) % 3] for j, c in enumerate(codes)]

        assert packer.pack(*values) == bytes(named_struct(cls, packer.fields, values)), pick


class Captured:

    def __init__(self):

        self.calls = []

    def entry(self, name):

        def call(packed):

            self.calls.append((name, packed))
            return _native.SS_OK

        return call


@pytest.fixture
def captured(monkeypatch):
    """The functional drivers on CPU tensors up to the library call, whose packed bytes it records."""

    cap = Captured()
    monkeypatch.setattr(_native, "packed_entry", cap.entry)
    monkeypatch.setattr(_native, "require_device", lambda *t: None)
    monkeypatch.setattr(_native, "stream_of", lambda t: 0x5EA3)

    return cap


def tensors(rows=6, vocab=9000, slots=8, target=12000, seed=0):

    g = torch.Generator().manual_seed(seed)
    words = -(-target // 32)

    return dict(
        logits=torch.randn(rows, vocab, generator=g).to(torch.bfloat16),
        indicators=torch.zeros(slots, dtype=torch.int16),
        grammar=torch.zeros(slots, words, dtype=torch.int32),
        context_counts=torch.zeros(slots, target, dtype=torch.int32),
        decode_counts=torch.zeros(slots, target + 4, dtype=torch.int32),
        repetition_penalties=torch.ones(slots), frequency_penalties=torch.zeros(slots),
        presence_penalties=torch.zeros(slots), logit_bias=torch.zeros(slots, target, dtype=torch.bfloat16),
        temperature=torch.ones(slots), top_k=torch.zeros(slots, dtype=torch.int32), top_p=torch.ones(slots),
        min_p=torch.zeros(slots), top_k_logprobs=torch.zeros(slots, dtype=torch.int32),
    )


def expected_fields(call, sel, t, scratch, stream=0x5EA3):
    """ss_singular_args by field name, as fused_singular must fill it for keyword set `call`."""

    a = lambda x: 0 if x is None else x.data_ptr()
    s = lambda x: 0 if x is None else x.stride(0)
    logits = t["logits"]
    lp = sel.logprobs
    top = lp.top_k if lp is not None else None
    philox = call.get("philox_seed")
    drafted = call.get("drafted_tokens")
    history = call.get("timestep", 0) if drafted is not None else 0
    world, shard = call.get("world_size", 1), call.get("shard_size") or logits.size(1)
    bias = t["logit_bias"]

    return dict(
        logits=a(logits), stride_logits=logits.stride(0), rows=logits.size(0), vocab_size=logits.size(1),
        target_vocab=call.get("target_vocab") or bias.size(-1), block_n=call.get("block_n", 4096),
        lookahead=call.get("lookahead", 0), timestep=history,
        max_top_logprobs=call.get("max_top_logprobs", 5) if top is not None else 0,
        is_prefill=int(call.get("is_prefill", False)), update_counts=int(call.get("update_counts", False)),
        return_logprobs=int(lp is not None), return_probabilities=int(sel.probabilities is not None),
        strategy=fs.KERNEL_LAYOUTS[call.get("kernel_layout")],
        indicators=a(t["indicators"]), slot_mapping=a(call.get("slot_mapping")), d2t=a(call.get("d2t_mapping")),
        grammar=a(t["grammar"]), stride_grammar=s(t["grammar"]),
        context_counts=a(t["context_counts"]), stride_context=s(t["context_counts"]),
        decode_counts=a(t["decode_counts"]), stride_decode=s(t["decode_counts"]),
        drafted_tokens=a(drafted) if history else 0, stride_drafted=s(drafted),
        repetition=a(t["repetition_penalties"]), frequency=a(t["frequency_penalties"]),
        presence=a(t["presence_penalties"]), logit_bias=a(bias), stride_bias=s(bias),
        temperature=a(t["temperature"]), top_k=a(t["top_k"]), top_p=a(t["top_p"]), min_p=a(t["min_p"]),
        top_logprobs=a(t["top_k_logprobs"]),
        gumbel=0 if philox is not None else a(call.get("gumbel_noise")),
        stride_gumbel=0 if philox is not None else s(call.get("gumbel_noise")),
        philox=_native.Philox(philox & (2 ** 64 - 1), call.get("philox_offset", 0) & 0xFFFFFFFF, 1)
        if philox is not None else _native.Philox(0, 0, 0),
        philox_step=call.get("philox_step", 0), stages=fs.STAGES[call.get("stage")],
        tokens=a(sel.tokens), stride_tokens=sel.tokens.stride(0),
        logprobs=a(lp.selected if lp is not None else None), stride_logprobs=s(lp.selected if lp is not None else None),
        top_values=a(top.logprobs if top is not None else None), top_tokens=a(top.tokens if top is not None else None),
        stride_top=s(top.logprobs if top is not None else None),
        probabilities=a(sel.probabilities), stride_probabilities=s(sel.probabilities),
        scratch=a(scratch), stride_scratch=s(scratch), stream=stream,
        world_size=world, local_rank=call.get("local_rank", 0), shard_size=shard,
    )


CALLS = {
    "decode, philox, logprobs": dict(philox_seed=2 ** 63 + 5, philox_offset=2 ** 33 + 7, return_logprobs=True,
                                     update_counts=True, max_top_logprobs=5),
    "prefill, noise plane, no logprobs": dict(is_prefill=True, noise=True, block_n=2048),
    "drafting, d2t, slots, history, probabilities": dict(drafting=True, lookahead=3, timestep=2, philox_seed=9,
                                                         philox_step=2, kernel_layout="rowwise", block_n=1024),
    "sharded tile stage": dict(world_size=4, local_rank=3, shard_size=9008, stage="tiles", philox_seed=1,
                               target_vocab=36032),
    "logprobs without a top list": dict(return_logprobs=True, max_top_logprobs=0, noise=True, stage="rows"),
}


@pytest.mark.parametrize("name", list(CALLS))
def test_fused_singular_packs_every_field_by_name(name, captured):

    call = dict(CALLS[name])
    t = tensors(seed=len(name))
    g = torch.Generator().manual_seed(1)
    rows, slots = t["logits"].size(0), t["indicators"].size(0)

    if call.pop("noise", False):

        call["gumbel_noise"] = torch.randn(slots, 9000, generator=g)

    if call.pop("drafting", False):

        call["slot_mapping"] = torch.randperm(slots, generator=g)[:rows].to(torch.int32)
        call["d2t_mapping"] = torch.randperm(12000, generator=g)[:9000].to(torch.int32)
        call["drafted_tokens"] = torch.randint(0, 12000, (rows, 4), generator=g).to(torch.int32)
        call["return_probabilities"] = True
        call["target_vocab"] = 12000

    world = call.get("world_size", 1)
    scratch = torch.empty(rows, world * -(-9000 // call.get("block_n", 4096)) * 128, dtype=torch.int32)
    sel = fs.fused_singular(**t, **call, scratchpad=scratch)

    assert len(captured.calls) == 1
    entry, packed = captured.calls[0]
    assert entry == "ss_fused_singular"
    assert packed == bytes(_native.SingularArgs(**expected_fields(call, sel, t, scratch)))


def test_static_scratch_takes_the_no_allocation_entry(captured):

    t = tensors()
    sel = fs.fused_singular(**t, philox_seed=3, static_scratch=True)
    entry, packed = captured.calls[0]

    assert entry == "ss_fused_singular_noalloc"
    assert packed == bytes(_native.SingularArgs(**expected_fields(dict(philox_seed=3), sel, t, None)))


def test_packed_entry_reads_the_bytes_as_the_struct():
    """Into the library's own argument checks (which return before any launch): the packed entry
    point answers every case as the ctypes entry point does."""

    lib = _native.load()
    packer = fs.SINGULAR_ARGS
    base = dict(logits=0x1000, stride_logits=8192, rows=4, vocab_size=8192, target_vocab=8192,
                block_n=1024, indicators=0x1000, tokens=0x1000, stride_tokens=1, scratch=0x10000,
                stride_scratch=8 * 128, philox_seed=1, philox_offset=0, philox_enabled=1)

    for change in (dict(block_n=512), dict(vocab_size=1024), dict(stride_scratch=100), dict(timestep=65),
                   dict(max_top_logprobs=129), dict(philox_enabled=0), dict(rows=0)):

        values = [dict(base, **change).get(f, 0) for f in packer.fields]
        args = named_struct(_native.SingularArgs, packer.fields, values)

        assert _native.packed_entry("ss_fused_singular")(packer.pack(*values)) == \
            lib.ss_fused_singular(ctypes.byref(args)), change


def multistep_expected(call, ver, t, flat, scratch, values, indices, uniform, stream=0x5EA3):
    """ss_multistep_args by field name, as fused_multistep must fill it for keyword set `call`."""

    a = lambda x: 0 if x is None else x.data_ptr()
    s = lambda x: 0 if x is None else x.stride(0)
    step = lambda x: 0 if x is None else (x.stride(1) if x.dim() >= 3 else 0)
    lp = ver.logprobs
    top = lp.top_k if lp is not None else None
    top_values = top.logprobs.flatten(0, -2) if top is not None else None
    philox = call.get("philox_seed")
    noise = call.get("gumbel_noise")

    return dict(
        logits=a(flat), stride_logits=flat.stride(0), rows=flat.size(0), batch=t["batch"],
        vocab_size=flat.size(1), block_n=call.get("block_n", 4096), lookahead=t["gamma"],
        max_top_logprobs=call.get("max_top_logprobs", 5) if top is not None else 0,
        update_counts=int(call.get("update_counts", False)), return_logprobs=int(lp is not None),
        cu_seqlens=a(call.get("cu_seqlens")), indicators=a(t["indicators"]), slot_mapping=a(call.get("slot_mapping")),
        drafted_tokens=a(t["drafted_tokens"]),
        grammar=a(t["grammar"]), grammar_stride_slot=s(t["grammar"]), grammar_stride_step=step(t["grammar"]),
        context_counts=a(t["context_counts"]), stride_context=s(t["context_counts"]),
        decode_counts=a(t["decode_counts"]), stride_decode=s(t["decode_counts"]),
        repetition=a(t["repetition_penalties"]), frequency=a(t["frequency_penalties"]),
        presence=a(t["presence_penalties"]), logit_bias=a(t["logit_bias"]), stride_bias=s(t["logit_bias"]),
        temperature=a(t["temperature"]), top_k=a(t["top_k"]), top_p=a(t["top_p"]), min_p=a(t["min_p"]),
        top_logprobs=a(t["top_k_logprobs"]),
        draft_probabilities=a(call.get("draft_probabilities")), probs_stride_slot=s(call.get("draft_probabilities")),
        probs_stride_step=step(call.get("draft_probabilities")),
        uniform=a(uniform), stride_uniform=s(uniform),
        gumbel=0 if philox is not None else a(noise), gumbel_stride_slot=0 if philox is not None else s(noise),
        gumbel_stride_step=0 if philox is not None else step(noise),
        philox=_native.Philox(philox & (2 ** 64 - 1), call.get("philox_offset", 0) & 0xFFFFFFFF, 1)
        if philox is not None else _native.Philox(0, 0, 0),
        out_tokens=a(ver.tokens), offsets=a(ver.offsets), logprobs=a(lp.selected if lp is not None else None),
        top_values=a(top_values), top_tokens=a(top.tokens if top is not None else None), stride_top=s(top_values),
        values=a(values), indices=a(indices), scratch=a(scratch), stride_scratch=scratch.stride(0), stream=stream,
        all_greedy=int(call.get("all_greedy", False)),
    )


MULTISTEP_CALLS = {
    "blocked, philox, logprobs, probabilities": dict(philox_seed=2 ** 64 - 3, philox_offset=2 ** 32 + 9,
                                                     return_logprobs=True, update_counts=True, probabilities=True),
    "varlen, slots, noise planes": dict(varlen=True, noise=True, slots=True, block_n=2048, max_top_logprobs=0,
                                        return_logprobs=True),
    "all greedy hint": dict(all_greedy=True, philox_seed=4, block_n=1024),
}


@pytest.mark.parametrize("name", list(MULTISTEP_CALLS))
def test_fused_multistep_packs_every_field_by_name(name, captured):

    from sonic_sampler.interface.functional import multistep as fm

    call = dict(MULTISTEP_CALLS[name])
    g = torch.Generator().manual_seed(len(name))
    batch, gamma, vocab, slots = 3, 2, 9000, 5
    n = gamma + 1
    t = tensors(rows=batch * n, vocab=vocab, slots=slots, target=vocab, seed=len(name))
    t.update(batch=batch, gamma=gamma)
    t["grammar"] = torch.zeros(slots, n, -(-vocab // 32), dtype=torch.int32)
    t["drafted_tokens"] = torch.randint(0, vocab, (batch * n,), generator=g).to(torch.int32)
    logits = t["logits"]

    if call.pop("varlen", False):

        call["cu_seqlens"] = torch.arange(0, batch * n + 1, n, dtype=torch.int32)
        call["lookahead"] = gamma

    else:

        logits = logits.view(batch, n, vocab)
        t["drafted_tokens"] = t["drafted_tokens"].view(batch, n)

    if call.pop("noise", False):

        call["gumbel_noise"] = torch.randn(slots, n, vocab, generator=g)
        call["uniform_noise"] = torch.rand(batch, gamma, generator=g)

    if call.pop("slots", False):

        call["slot_mapping"] = torch.randperm(slots, generator=g)[:batch].to(torch.int32)

    if call.pop("probabilities", False):

        call["draft_probabilities"] = torch.rand(slots, gamma, vocab, generator=g).to(torch.bfloat16)

    flat = t["logits"]
    scratch = torch.empty(batch * n, -(-vocab // call.get("block_n", 4096)) * 128, dtype=torch.int32)
    values = torch.empty(batch * n, 128)
    indices = torch.empty(batch * n, 128, dtype=torch.int32)
    uniform = call.get("uniform_noise")

    if uniform is None:

        uniform = torch.rand(batch, gamma)
        call["uniform_noise"] = uniform

    kw = {k: v for k, v in t.items() if k not in ("batch", "gamma", "logits")}
    ver = fm.fused_multistep(logits=logits, **kw, **call, scratchpad=scratch, values=values, indices=indices)

    assert len(captured.calls) == 1
    entry, packed = captured.calls[0]
    assert entry == "ss_fused_multistep"
    assert packed == bytes(_native.MultistepArgs(**multistep_expected(call, ver, t, flat, scratch, values, indices,
                                                                     uniform)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bounded_topk_packs_every_field_by_name(dtype, captured):

    from sonic_sampler.interface import UnshardedBoundedTopK

    topk = UnshardedBoundedTopK.initialize(vocab_size=9000, batch_size=6, k=32, block_size=2048, device="cpu")
    logits = torch.randn(2, 3, 9000).to(dtype)
    topk(logits)

    wide = dtype == torch.float32
    scratch, values = topk._wide_buffers(6) if wide else (topk.scratchpad, topk.values)
    flat = logits.flatten(0, 1)
    expected = _native.TopKArgs(
        logits=flat.data_ptr(), stride_logits=flat.stride(0),
        dtype=_native.SS_DTYPE_F32 if wide else _native.SS_DTYPE_BF16, rows=6, vocab_size=9000, k=32,
        block_n=2048, strategy=0, scratch=scratch.data_ptr(), stride_scratch=scratch.stride(0),
        values=values.data_ptr(), indices=topk.indices.data_ptr(), stream=0x5EA3)

    assert captured.calls == [("ss_topk", bytes(expected))]


def test_undersized_probability_buffers_are_rejected(captured):
    """A draft-probability buffer is addressed by slot: one whose storage does not reach the last
    slot it may be indexed by raises before any launch, while a strided view of a buffer that does
    (an engine's `draft_probs[:rows, t]`) passes."""

    from sonic_sampler.interface.functional import multistep as fm

    t = tensors(rows=6, vocab=9000, slots=8, target=12000)
    g = torch.Generator().manual_seed(3)
    slot_mapping = torch.randperm(8, generator=g)[:6].to(torch.int32)
    d2t = torch.randperm(12000, generator=g)[:9000].to(torch.int32)
    call = dict(slot_mapping=slot_mapping, d2t_mapping=d2t, target_vocab=12000, return_probabilities=True,
                philox_seed=1, drafted_tokens=torch.zeros(6, 4, dtype=torch.int32), timestep=1, lookahead=3)

    with pytest.raises(ValueError, match="does not cover"):

        fs.fused_singular(**t, **call, draft_probabilities=torch.zeros(6, 3, 12000, dtype=torch.bfloat16)[:, 1])

    fs.fused_singular(**t, **call, draft_probabilities=torch.zeros(8, 3, 12000, dtype=torch.bfloat16)[:6, 1])
    assert len(captured.calls) == 1

    # the verifier reads [slot, step, token] of every step of the lookahead
    batch, gamma, vocab = 3, 2, 9000
    v = tensors(rows=batch * (gamma + 1), vocab=vocab, slots=5, target=vocab)
    v["grammar"] = torch.zeros(5, gamma + 1, -(-vocab // 32), dtype=torch.int32)
    logits = v.pop("logits").view(batch, gamma + 1, vocab)
    drafted = torch.zeros(batch, gamma + 1, dtype=torch.int32)
    base = dict(logits=logits, drafted_tokens=drafted, uniform_noise=torch.rand(batch, gamma), philox_seed=2,
                slot_mapping=torch.tensor([4, 0, 2], dtype=torch.int32), **v)

    with pytest.raises(ValueError, match="does not cover"):

        fm.fused_multistep(**base, draft_probabilities=torch.zeros(3, gamma, vocab, dtype=torch.bfloat16))

    with pytest.raises(ValueError, match="does not cover"):

        fm.fused_multistep(**base, draft_probabilities=torch.zeros(5, gamma - 1, vocab, dtype=torch.bfloat16))

    fm.fused_multistep(**base, draft_probabilities=torch.zeros(5, gamma, vocab, dtype=torch.bfloat16))
    assert len(captured.calls) == 2
