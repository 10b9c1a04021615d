"""Tuned dispatch tables (reference ``interface/dispatch.py:36-268``).

A table maps a vocabulary bucket to batch buckets, each holding a priority-ordered list of
launch configurations, in the reference's TOML schema. The tables shipped here are for gfx950
(``resources/dispatch/gfx950_k128.toml``). ``arch`` may be given as ``950`` or ``"gfx950"``; when
it is omitted the current device's architecture is used. Call kinds whose best tile widths differ
from the fused single step's have tables of their own beside it (``gfx950_k128_multistep.toml``,
``gfx950_k128_drafting.toml``, ``gfx950_k128_topk.toml``): the verification without penalties is
bound by per-element instructions and prefers wider tiles than the decode step, which reads four
planes per element. A kind without a table, or without a bucket for a vocabulary, uses the shared
table. The warp counts and top-k strategy of
each entry are kept for schema compatibility; the gfx950 kernels use one 256-thread workgroup
shape and one selection algorithm, so only ``block_n`` changes what runs.
"""

from __future__ import annotations

from bisect import bisect_left
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass, field
from importlib import resources
from pathlib import Path
from typing import Dict, List, Literal, Optional, Union

import tomli

import torch

from sonic_sampler.ops.base import MAX_K, next_power_of_2


Strategy = Literal["bitonic", "adaptive", "radix"]


class DispatchContext:

    def __init__(self) -> None:

        self.value: ContextVar[bool] = ContextVar("inference", default=False)

    @property
    def is_inference(self) -> bool:

        return self.value.get()

    @contextmanager
    def __call__(self, *, inference: bool = True):

        token = self.value.set(inference)

        try:

            yield

        finally:

            self.value.reset(token)


DISPATCH_CONTEXT = DispatchContext()


@dataclass(eq=True)
class TwoStageWarpConfig:

    first: int
    second: int

    @classmethod
    def default(cls) -> "TwoStageWarpConfig":

        return TwoStageWarpConfig(first=16, second=8)


@dataclass(eq=True)
class ThreeStageWarpConfig(TwoStageWarpConfig):

    # The verification stage's warp count.
    third: int = 0

    @property
    def two_stage(self) -> TwoStageWarpConfig:

        return TwoStageWarpConfig(first=self.first, second=self.second)

    @classmethod
    def from_config(cls, config: TwoStageWarpConfig, third: Optional[int] = None,
                    gamma: int = 3) -> "ThreeStageWarpConfig":

        return ThreeStageWarpConfig(first=config.first, second=config.second,
                                    third=third or next_power_of_2(gamma + 1))

    @classmethod
    def default(cls, gamma: int = 3) -> "ThreeStageWarpConfig":

        return cls.from_config(config=TwoStageWarpConfig.default(), gamma=gamma)


@dataclass
class RuntimeConfig:

    priority: int
    block_n: int
    strategy: Strategy
    first_warps: int
    second_warps: int

    @property
    def warp_config(self) -> TwoStageWarpConfig:

        return TwoStageWarpConfig(first=self.first_warps, second=self.second_warps)


class PriorityBucket(list):

    def get(self, size: int, margin: float = 0.5):
        """The first bucket whose size is >= `size`, else the last if within (1 + margin)."""

        index = bisect_left([b.size for b in self], size)

        if index < len(self):

            return self[index]

        if self and size < self[-1].size * (1 + margin):

            return self[-1]

        return None


@dataclass
class BatchBucket:

    size: int
    config: List[RuntimeConfig]
    mapping: Dict[str, RuntimeConfig] = field(default_factory=dict)

    def __post_init__(self) -> None:

        if DISPATCH_CONTEXT.is_inference:

            self.mapping = {c.strategy: c for c in self.config}

    @property
    def best(self) -> RuntimeConfig:

        return self.config[0]

    def get(self, strategy: str) -> RuntimeConfig:

        return self.mapping[strategy]


@dataclass
class VocabBucket:

    size: int
    batch: PriorityBucket

    @property
    def block_n(self) -> int:

        return min(c.block_n for b in self.batch for c in b.config)


@dataclass
class DispatchMetadata:

    version: int
    timestamp: str


def resolve_arch(arch: Union[int, str, None]) -> str:
    """Table key for an architecture: ``950`` / ``"gfx950"`` -> ``"gfx950"``; ``None`` -> device."""

    if arch is None:

        if not torch.cuda.is_available():

            return "gfx950"

        name = torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName

        return name.split(":")[0]

    if isinstance(arch, int):

        return f"gfx{arch}"

    return arch if arch.startswith(("gfx", "sm")) else f"gfx{arch}"


@dataclass
class DispatchSummary:

    metadata: DispatchMetadata
    k: int
    vocab: PriorityBucket

    @classmethod
    def from_dict(cls, data: dict) -> "DispatchSummary":

        vocab = PriorityBucket(
            VocabBucket(
                size=v["size"],
                batch=PriorityBucket(
                    BatchBucket(size=b["size"], config=[RuntimeConfig(**c) for c in b["config"]])
                    for b in v["batch"]
                ),
            )
            for v in data["vocab"]
        )

        return cls(metadata=DispatchMetadata(**data["metadata"]), k=data["k"], vocab=vocab)

    @classmethod
    def read(cls, path, inference: bool = True) -> "DispatchSummary":

        with DISPATCH_CONTEXT(inference=inference):

            return cls.from_dict(tomli.loads(Path(path).read_text() if not hasattr(path, "read_text")
                                             else path.read_text()))

    @classmethod
    def load(cls, k: int = MAX_K, arch: Union[int, str, None] = None, inference: bool = True,
             kind: Optional[str] = None) -> Optional["DispatchSummary"]:
        """The shipped table ``{arch}_k{k}.toml``, or with `kind` the table of that call kind
        (``{arch}_k{k}_{kind}.toml``), None where there is no such file."""

        name = f"{resolve_arch(arch)}_k{k}" + (f"_{kind}" if kind else "")
        path = resources.files("sonic_sampler") / "resources/dispatch" / f"{name}.toml"

        if path.is_file():

            return cls.read(path, inference=inference)

        return None

    @classmethod
    def default(cls) -> Optional["DispatchSummary"]:

        return cls.load(k=MAX_K, arch="gfx950")

    def to_toml(self) -> str:

        lines = [f"k = {self.k}", "", "[metadata]", f"version = {self.metadata.version}",
                 f'timestamp = "{self.metadata.timestamp}"', ""]

        for v in self.vocab:

            lines += ["[[vocab]]", f"size = {v.size}", ""]

            for b in v.batch:

                lines += ["[[vocab.batch]]", f"size = {b.size}", "config = ["]

                for c in b.config:

                    lines.append(
                        f'    {{ priority = {c.priority}, block_n = {c.block_n}, strategy = "{c.strategy}", '
                        f"first_warps = {c.first_warps}, second_warps = {c.second_warps} }},"
                    )

                lines += ["]", ""]

        return "\n".join(lines)

    def save(self, path) -> None:

        Path(path).resolve().write_text(self.to_toml())
