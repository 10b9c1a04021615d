"""The C-ABI library on the CPU: it loads, exports every entry point the header declares, agrees
with the Python struct mirrors, and rejects invalid arguments before touching a device."""

from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess
import sys

from pathlib import Path

import pytest

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

from sonic_sampler import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sonic_sampler.h"


def header_text() -> str:

    return HEADER.read_text()


def declared_functions() -> list[str]:

    # return type, optional pointer star, ss_ name, opening parenthesis
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ss_\w+)\s*\(", header_text(), re.M)))


def header_constant(name: str) -> int:

    match = re.search(rf"#define\s+{name}\s+(\d+)", header_text())
    assert match, name

    return int(match.group(1))


def test_header_declares_the_entry_points():

    names = declared_functions()

    for required in ("ss_topk", "ss_fused_singular", "ss_fused_multistep", "ss_indexed_copy", "ss_gumbel_materialize",
                     "ss_philox_raw", "ss_abi_version", "ss_status_string", "ss_args_size"):

        assert required in names


def test_library_exports_every_declared_symbol():

    lib = _native.load()

    for name in declared_functions():

        assert hasattr(lib, name), f"{name} declared in include/sonic_sampler.h but not exported"


def test_abi_version_and_struct_sizes():

    lib = _native.load()

    assert lib.ss_abi_version() == header_constant("SS_ABI_VERSION") == _native.ABI_VERSION
    assert lib.ss_args_size(0) == ctypes.sizeof(_native.TopKArgs)
    assert lib.ss_args_size(1) == ctypes.sizeof(_native.SingularArgs)
    assert lib.ss_args_size(2) == ctypes.sizeof(_native.MultistepArgs)
    assert lib.ss_args_size(3) == ctypes.sizeof(_native.IndexedCopyArgs)
    assert lib.ss_args_size(4) == -1


C_STRUCTS = {"ss_philox": _native.Philox, "ss_topk_args": _native.TopKArgs,
             "ss_singular_args": _native.SingularArgs, "ss_multistep_args": _native.MultistepArgs,
             "ss_indexed_copy_args": _native.IndexedCopyArgs}


@pytest.mark.parametrize("compiler,std", [("gcc", "-std=c99"), ("g++", "-std=c++11")])
def test_header_layout_is_the_mirrors_layout(tmp_path, compiler, std):
    """The header compiles alone as strict C99 and as C++11, and the compiler places every field
    of every argument struct at the offset, and with the size, that the ctypes mirrors give it.
    The struct sizes the library reports cannot tell two swapped fields of one size apart."""

    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} is not installed")

    prints = []

    for cname, cls in C_STRUCTS.items():
        prints.append(f'printf("{cname} %zu %zu\\n", (size_t)0, sizeof({cname}));')

        for name, _ in cls._fields_:
            prints.append(f'printf("{cname}.{name} %zu %zu\\n", offsetof({cname}, {name}), '
                          f'sizeof((({cname} *)0)->{name}));')

    source = tmp_path / ("layout.c" if compiler == "gcc" else "layout.cpp")
    source.write_text("#include <stddef.h>\n#include <stdio.h>\n#include \"sonic_sampler.h\"\n"
                      "int main(void) {\n" + "\n".join(prints) + "\nreturn 0;\n}\n")
    exe = tmp_path / "layout"
    build = subprocess.run([compiler, std, "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", str(HEADER.parent),
                            str(source), "-o", str(exe)], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr

    placed = {}

    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        name, offset, size = line.split()
        placed[name] = (int(offset), int(size))

    for cname, cls in C_STRUCTS.items():
        assert placed[cname] == (0, ctypes.sizeof(cls)), cname

        for name, _ in cls._fields_:
            field = getattr(cls, name)
            assert placed[f"{cname}.{name}"] == (field.offset, field.size), f"{cname}.{name}"


def test_status_strings():

    lib = _native.load()
    expected = {0: b"ok", 1: b"invalid argument", 2: b"unsupported configuration", 3: b"kernel launch failed"}

    for code, text in expected.items():

        assert lib.ss_status_string(code) == text

    assert lib.ss_status_string(99) == b"unknown status"


def test_null_arguments_are_rejected():

    lib = _native.load()

    assert lib.ss_topk(None) == 1
    assert lib.ss_fused_singular(None) == 1
    assert lib.ss_fused_multistep(None) == 1


def fake(address: int = 0x1000) -> int:
    """A non-null pointer that is never dereferenced: every call below returns before any launch."""

    return address


def singular_args(**overrides) -> _native.SingularArgs:

    fields = dict(logits=fake(), stride_logits=8192, rows=4, vocab_size=8192, target_vocab=8192,
                  block_n=1024, indicators=fake(), tokens=fake(), stride_tokens=1,
                  scratch=fake(0x10000), stride_scratch=8 * 128, philox=_native.Philox(1, 0, 1))
    fields.update(overrides)

    return _native.SingularArgs(**fields)


@pytest.mark.parametrize("overrides, status", [
    (dict(block_n=512), 2),                      # tile width not compiled
    (dict(vocab_size=1024), 1),                  # a single tile
    (dict(stride_scratch=100), 1),               # scratch row too short for tiles * 128
    (dict(scratch=fake(0x10004)), 1),            # scratch not 16-byte aligned
    (dict(stride_logits=100), 1),                # logits row shorter than the vocabulary
    (dict(timestep=65), 1),                      # history longer than a wave can stage
    (dict(max_top_logprobs=129), 1),             # Z above 128
    (dict(philox=_native.Philox(1, 0, 0)), 1),   # neither Philox nor a noise plane
    (dict(rows=0), 0),                           # empty batch: nothing to launch
])
def test_singular_validation(overrides, status):

    lib = _native.load()

    assert lib.ss_fused_singular(ctypes.byref(singular_args(**overrides))) == status


def test_multistep_validation():

    lib = _native.load()
    base = dict(logits=fake(), stride_logits=8192, rows=10, batch=2, vocab_size=8192, block_n=1024,
                lookahead=4, indicators=fake(), drafted_tokens=fake(), out_tokens=fake(), offsets=fake(),
                values=fake(), indices=fake(), scratch=fake(0x10000), stride_scratch=8 * 128,
                uniform=fake(), philox=_native.Philox(1, 0, 1))

    assert lib.ss_fused_multistep(ctypes.byref(_native.MultistepArgs(**dict(base, block_n=3000)))) == 2
    assert lib.ss_fused_multistep(ctypes.byref(_native.MultistepArgs(**dict(base, uniform=None)))) == 1
    assert lib.ss_fused_multistep(ctypes.byref(_native.MultistepArgs(**dict(base, rows=7)))) == 1  # not B * (gamma + 1)
    assert lib.ss_fused_multistep(ctypes.byref(_native.MultistepArgs(**dict(base, lookahead=64, rows=130)))) == 1
    assert lib.ss_fused_multistep(ctypes.byref(_native.MultistepArgs(**dict(base, rows=0, batch=0)))) == 0


def test_topk_validation():

    lib = _native.load()
    base = dict(logits=fake(), stride_logits=32000, dtype=1, rows=8, vocab_size=32000, k=32, block_n=2048,
                scratch=fake(), stride_scratch=16 * 32, values=fake(), indices=fake())

    assert lib.ss_topk(ctypes.byref(_native.TopKArgs(**dict(base, k=48)))) == 1      # not a power of 2
    assert lib.ss_topk(ctypes.byref(_native.TopKArgs(**dict(base, k=256)))) == 1     # above 128
    assert lib.ss_topk(ctypes.byref(_native.TopKArgs(**dict(base, dtype=7)))) == 2   # unknown dtype
    assert lib.ss_topk(ctypes.byref(_native.TopKArgs(**dict(base, rows=0)))) == 0


def test_noise_validation():

    lib = _native.load()

    assert lib.ss_gumbel_materialize(1, 0, -1, 1, 10, fake(), 10, 10, None) == 1
    assert lib.ss_gumbel_materialize(1, 0, 1, 1, 10, None, 10, 10, None) == 1
    assert lib.ss_gumbel_materialize(1, 0, 2, 2, 10, fake(), 10, 5, None) == 1   # overlapping rows
    assert lib.ss_gumbel_materialize(1, 0, 0, 1, 10, fake(), 10, 10, None) == 0  # nothing to do
    assert lib.ss_philox_raw(1, 0, 1, 1, -5, fake(), None) == 1


def test_missing_library_fails_loudly():
    """Without the built library the product path raises instead of falling back."""

    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import torch\n"
        "from sonic_sampler import _native\n"
        "try:\n"
        "    _native.load()\n"
        "except RuntimeError as e:\n"
        "    print('raised', e)\n"
    ) % str(ROOT / "sonic-sampler_amd")
    env = dict(os.environ, SONIC_SAMPLER_LIB=str(ROOT / "does-not-exist.so"))
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)

    assert "raised" in out.stdout, out.stdout + out.stderr
