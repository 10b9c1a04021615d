"""ctypes binding of the gfx950 HIP library (C-ABI declared in ``include/sonic_sampler.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch already mapped
(both carry the soname ``libamdhip64.so.7``), which makes torch's stream handles valid inside it.
There is deliberately no CPU fallback: if the library is missing every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import struct
from pathlib import Path

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libsonic_sampler.so"

c_p = ctypes.c_void_p
c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_u32 = ctypes.c_uint32
c_u64 = ctypes.c_uint64

SS_OK = 0
SS_ERR_SCRATCH_LIMIT = 4
STRATEGY_AUTO, STRATEGY_TILES, STRATEGY_ROWWISE = 0, 1, 2
STAGE_TILES, STAGE_ROWS = 1, 2
STATIC_SCRATCH_BYTES = 8 << 20   # SS_STATIC_SCRATCH_BYTES
SS_DTYPE_BF16 = 0
SS_DTYPE_F32 = 1
ABI_VERSION = 3


class Philox(ctypes.Structure):
    _fields_ = [("seed", c_u64), ("offset", c_u32), ("enabled", c_i32)]


class TopKArgs(ctypes.Structure):
    _fields_ = [
        ("logits", c_p), ("stride_logits", c_i64), ("dtype", c_i32), ("rows", c_i32),
        ("vocab_size", c_i32), ("k", c_i32), ("block_n", c_i32), ("strategy", c_i32),
        ("scratch", c_p), ("stride_scratch", c_i64), ("values", c_p),
        ("indices", c_p), ("stream", c_p),
    ]


class SingularArgs(ctypes.Structure):
    _fields_ = [
        ("logits", c_p), ("stride_logits", c_i64), ("rows", c_i32), ("vocab_size", c_i32),
        ("target_vocab", c_i32), ("block_n", c_i32), ("lookahead", c_i32), ("timestep", c_i32),
        ("max_top_logprobs", c_i32), ("is_prefill", c_i32), ("update_counts", c_i32),
        ("return_logprobs", c_i32), ("return_probabilities", c_i32), ("strategy", c_i32),
        ("indicators", c_p), ("slot_mapping", c_p), ("d2t", c_p),
        ("grammar", c_p), ("stride_grammar", c_i64),
        ("context_counts", c_p), ("stride_context", c_i64),
        ("decode_counts", c_p), ("stride_decode", c_i64),
        ("drafted_tokens", c_p), ("stride_drafted", c_i64),
        ("repetition", c_p), ("frequency", c_p), ("presence", c_p),
        ("logit_bias", c_p), ("stride_bias", c_i64),
        ("temperature", c_p), ("top_k", c_p), ("top_p", c_p), ("min_p", c_p),
        ("top_logprobs", c_p), ("gumbel", c_p), ("stride_gumbel", c_i64),
        ("philox", Philox), ("philox_step", c_i32), ("stages", c_i32),
        ("tokens", c_p), ("stride_tokens", c_i64),
        ("logprobs", c_p), ("stride_logprobs", c_i64),
        ("top_values", c_p), ("top_tokens", c_p), ("stride_top", c_i64),
        ("probabilities", c_p), ("stride_probabilities", c_i64),
        ("scratch", c_p), ("stride_scratch", c_i64), ("stream", c_p),
        ("tile_start", c_p), ("tile_end", c_p),
        ("world_size", c_i32), ("local_rank", c_i32), ("shard_size", c_i32), ("reserved", c_i32),
    ]


class MultistepArgs(ctypes.Structure):
    _fields_ = [
        ("logits", c_p), ("stride_logits", c_i64), ("rows", c_i32), ("batch", c_i32),
        ("vocab_size", c_i32), ("block_n", c_i32), ("lookahead", c_i32),
        ("max_top_logprobs", c_i32), ("update_counts", c_i32), ("return_logprobs", c_i32),
        ("cu_seqlens", c_p), ("indicators", c_p), ("slot_mapping", c_p), ("drafted_tokens", c_p),
        ("grammar", c_p), ("grammar_stride_slot", c_i64), ("grammar_stride_step", c_i64),
        ("context_counts", c_p), ("stride_context", c_i64),
        ("decode_counts", c_p), ("stride_decode", c_i64),
        ("repetition", c_p), ("frequency", c_p), ("presence", c_p),
        ("logit_bias", c_p), ("stride_bias", c_i64),
        ("temperature", c_p), ("top_k", c_p), ("top_p", c_p), ("min_p", c_p),
        ("top_logprobs", c_p),
        ("draft_probabilities", c_p), ("probs_stride_slot", c_i64), ("probs_stride_step", c_i64),
        ("uniform", c_p), ("stride_uniform", c_i64),
        ("gumbel", c_p), ("gumbel_stride_slot", c_i64), ("gumbel_stride_step", c_i64),
        ("philox", Philox),
        ("out_tokens", c_p), ("offsets", c_p), ("logprobs", c_p),
        ("top_values", c_p), ("top_tokens", c_p), ("stride_top", c_i64),
        ("values", c_p), ("indices", c_p),
        ("scratch", c_p), ("stride_scratch", c_i64), ("stream", c_p),
        ("tile_start", c_p), ("tile_end", c_p), ("all_greedy", c_i32),
    ]


class IndexedCopyArgs(ctypes.Structure):
    _fields_ = [
        ("source", c_p), ("stride_source", c_i64), ("target", c_p), ("stride_target", c_i64),
        ("indices", c_p), ("indicators", c_p), ("cols", c_i64), ("count", c_i32), ("slots", c_i32),
        ("stream", c_p),
    ]


_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    return Path(os.environ.get("SONIC_SAMPLER_LIB", _LIB_PATH))


def load() -> ctypes.CDLL:
    """Loads (once) and returns the HIP library; raises if it is absent or mismatched."""

    global _lib

    if _lib is not None:
        return _lib

    path = library_path()

    if not path.is_file():
        raise RuntimeError(
            f"sonic_sampler HIP library not found at {path}; build it with "
            "`python sonic-sampler_amd/build_native.py` (no CPU fallback exists)"
        )

    lib = ctypes.CDLL(str(path))

    lib.ss_abi_version.restype = c_i32
    lib.ss_status_string.restype = ctypes.c_char_p
    lib.ss_status_string.argtypes = [c_i32]
    lib.ss_args_size.restype = c_i64
    lib.ss_args_size.argtypes = [c_i32]

    for name, struct in (("ss_topk", TopKArgs), ("ss_fused_singular", SingularArgs),
                         ("ss_fused_singular_noalloc", SingularArgs),
                         ("ss_fused_multistep", MultistepArgs), ("ss_indexed_copy", IndexedCopyArgs)):
        fn = getattr(lib, name)
        fn.restype = c_i32
        fn.argtypes = [ctypes.POINTER(struct)]

    lib.ss_gumbel_materialize.restype = c_i32
    lib.ss_gumbel_materialize.argtypes = [c_u64, c_u32, c_i32, c_i32, c_i32, c_p, c_i64, c_i64, c_p]
    lib.ss_philox_raw.restype = c_i32
    lib.ss_philox_raw.argtypes = [c_u64, c_u32, c_i32, c_i32, c_i32, c_p, c_p]

    if lib.ss_abi_version() != ABI_VERSION:
        raise RuntimeError(f"sonic_sampler ABI mismatch: library {lib.ss_abi_version()}, "
                           f"bindings {ABI_VERSION}")

    for which, struct in enumerate((TopKArgs, SingularArgs, MultistepArgs, IndexedCopyArgs)):
        if lib.ss_args_size(which) != ctypes.sizeof(struct):
            raise RuntimeError(f"sonic_sampler ABI mismatch in {struct.__name__}: "
                               f"{lib.ss_args_size(which)} != {ctypes.sizeof(struct)} bytes")

    _lib = lib

    return lib


def check(status: int, what: str) -> None:

    if status != SS_OK:

        message = load().ss_status_string(status).decode()

        raise RuntimeError(f"{what} failed: {message} (status {status})")


def ptr(tensor: torch.Tensor | None) -> int | None:

    return None if tensor is None else tensor.data_ptr()


def addr(tensor: torch.Tensor | None) -> int:
    """A tensor's device address, 0 for an absent one (a field of a packed argument struct)."""

    return 0 if tensor is None else tensor.data_ptr()


def stride0(tensor: torch.Tensor | None) -> int:

    return 0 if tensor is None else tensor.stride(0)


# torch's current stream of a device index as the raw hipStream_t, without building a Stream
# object (about a fifteenth of the cost of torch.cuda.current_stream(device).cuda_stream)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(tensor: torch.Tensor) -> int:
    """torch's current stream on the tensor's device (a CUDA tensor's)."""

    if _raw_stream is not None:

        return _raw_stream(tensor.get_device())

    return torch.cuda.current_stream(tensor.device).cuda_stream


_CODES = {ctypes.c_void_p: "Q", ctypes.c_int32: "i", ctypes.c_uint32: "I", ctypes.c_int64: "q",
          ctypes.c_uint64: "Q"}


def _flat_layout(cls, base: int = 0, prefix: str = "") -> list:
    """(name, offset, size, struct code) of every scalar field of a ctypes struct in declaration
    order; a nested struct's fields stand in its place, named <field>_<member>."""

    layout = []

    for name, typ in cls._fields_:

        offset = getattr(cls, name).offset + base

        if isinstance(typ, type) and issubclass(typ, ctypes.Structure):

            layout += _flat_layout(typ, offset, f"{prefix}{name}_")

        else:

            layout.append((prefix + name, offset, ctypes.sizeof(typ), _CODES[typ]))

    return layout


class Packer:
    """The bytes of a ctypes argument struct from its field values given positionally, in
    declaration order (a nested struct's members in its place, pointers as integers, 0 for NULL):
    one ``struct.Struct.pack`` instead of the keyword constructor, about a sixth of its cost on a
    call's host path. ``fields`` lists the positions' names."""

    def __init__(self, cls):

        fmt, end = "<", 0

        for _, offset, size, code in _flat_layout(cls):

            fmt += f"{offset - end}x{code}" if offset > end else code
            end = offset + size

        fmt += f"{ctypes.sizeof(cls) - end}x" if ctypes.sizeof(cls) > end else ""
        self.fields = tuple(name for name, *_ in _flat_layout(cls))
        self.struct = struct.Struct(fmt)
        self.pack = self.struct.pack

        if self.struct.size != ctypes.sizeof(cls):

            raise RuntimeError(f"packed layout of {cls.__name__} is {self.struct.size} bytes, "
                               f"the struct {ctypes.sizeof(cls)}")


_packed_entries: dict = {}


def packed_entry(name: str):
    """Entry point `name` taking its argument struct as packed bytes (``Packer.pack``) instead of
    a ctypes struct: a function pointer of its own, apart from ``load().<name>``."""

    fn = _packed_entries.get(name)

    if fn is None:

        fn = load()[name]
        fn.restype = c_i32
        fn.argtypes = [ctypes.c_char_p]
        _packed_entries[name] = fn

    return fn


def event_handle(event: "torch.cuda.Event | None") -> int | None:
    """The hipEvent_t behind a torch event (created on first use), or None."""

    if event is None:

        return None

    if not event.cuda_event:

        event.record()

    return event.cuda_event


def event_pair(events) -> tuple:
    """(start, end) hipEvent_t handles of a pair of torch events, or (None, None)."""

    if events is None:

        return None, None

    start, end = events

    return event_handle(start), event_handle(end)


def require_device(*tensors: torch.Tensor | None) -> None:

    for tensor in tensors:

        if tensor is not None and tensor.device.type != "cuda":

            raise ValueError(
                f"sonic_sampler kernels run on the GPU only; got a tensor on {tensor.device}"
            )


def indexed_copy(source: torch.Tensor, target: torch.Tensor, indices: torch.Tensor,
                 indicators: torch.Tensor | None) -> None:
    """ss_indexed_copy over bf16 rows: target[i] = source[i] for every i in `indices` whose
    indicator is stochastic (bit 0x40 clear), on the current stream."""

    require_device(source, target, indices, indicators)

    if source.dtype != torch.bfloat16 or target.dtype != torch.bfloat16:
        raise ValueError("indexed_copy copies bfloat16 rows")

    src, dst = source.flatten(1), target.flatten(1)

    if src.stride(-1) != 1 or dst.stride(-1) != 1 or src.size(1) != dst.size(1) or src.size(0) != dst.size(0):
        raise ValueError("indexed_copy needs equally shaped source and target with contiguous rows")

    idx = indices.to(torch.int64).contiguous()
    args = IndexedCopyArgs(
        source=src.data_ptr(), stride_source=src.stride(0), target=dst.data_ptr(), stride_target=dst.stride(0),
        indices=idx.data_ptr(), indicators=None if indicators is None else indicators.data_ptr(),
        cols=src.size(1), count=idx.numel(), slots=src.size(0), stream=stream_of(src),
    )
    check(load().ss_indexed_copy(ctypes.byref(args)), "ss_indexed_copy")
