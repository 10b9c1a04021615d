"""Writes the golden fixtures of tests/golden/ from the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Usage: ``python tests/golden/make_fixtures.py [--out DIR]`` (from the repository root; DIR defaults
to this folder); ``--inputs CASE --out FILE`` writes one case's input tensors instead, which is how
the tests obtain the exact inputs (``fixture_inputs``). Each fixture is one
JSON file holding a small seeded case of one configuration shape, the SHA-256 of every input
tensor the case's generator produced (so a test can prove it feeds exactly those inputs), and the
oracle's outputs on them. The oracle runs with ``ATEN_CPU_CAPABILITY=default`` and one thread, so
the outputs do not depend on the host's vector units or thread count. The reference cannot be
imported here (it needs Python >= 3.12 and an NVIDIA GPU) and holds no golden vectors of its own,
so these outputs are the build's oracle's: they pin the oracle against drift and give the GPU
tests committed data to meet.

Cases (generators of bench.py at reduced sizes):
  singular   config-1 shape: autoregressive, every processor, top-k/p/min-p, logprobs + top-5
  drafting   config-4 shape: d2t 2000 -> 16384, grammar, 24 of 48 slots, probabilities
  multistep  config-3 shape: stochastic varlen verification, draft probabilities, top-20
  topk       config-0 shape: bounded top-k of fp32 rows, k = 32
"""

from __future__ import annotations

import os

os.environ.setdefault("ATEN_CPU_CAPABILITY", "default")

import hashlib  # noqa: E402
import json  # noqa: E402
import sys  # noqa: E402

from pathlib import Path  # noqa: E402

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent

for p in (ROOT, ROOT / "sonic-sampler_amd"):

    if str(p) not in sys.path:

        sys.path.insert(0, str(p))

import torch  # noqa: E402

# Case parameters. The tests regenerate each case's inputs from these and compare their digests.
SINGULAR = {"seed": 2001, "batch": 8, "vocab": 5000}
DRAFTING = {"seed": 2004, "rows": 24, "slots": 48, "gamma": 4, "draft_vocab": 2000, "target_vocab": 16384,
            "timestep": 2}
MULTISTEP = {"seed": 2003, "batch": 8, "gamma": 7, "vocab": 5000}
TOPK = {"seed": 2000, "rows": 4, "vocab": 3000, "k": 32}


def digest(t: torch.Tensor) -> str:
    """SHA-256 of a tensor's dtype, shape and bytes."""

    t = t.detach().contiguous().cpu()
    h = hashlib.sha256(f"{t.dtype}{tuple(t.shape)}".encode())
    h.update(t.view(torch.uint8).numpy().tobytes() if t.numel() else b"")

    return h.hexdigest()


# State members a case's path does not read (their planes may hold uninitialized memory)
UNREAD = {"singular": ("gumbel_draft", "uniform"), "drafting": ("gumbel_target", "uniform"),
          "multistep": ("gumbel_draft",)}


def state_digests(buffers, case: str) -> dict:
    """Digests of the SamplingBuffers members the case's path reads, as the oracle's State holds
    them (indicator lists as int32 tensors)."""

    import dataclasses

    from oracle import sampler as oracle

    st = oracle.State.from_buffers(buffers)
    out = {}

    for f in dataclasses.fields(st):

        if f.name in UNREAD[case]:

            continue

        v = getattr(st, f.name)
        out[f.name] = digest(torch.tensor(v, dtype=torch.int32) if isinstance(v, list) else v)

    return out


def singular_inputs():
    from bench import c1_workload

    return c1_workload(seed=SINGULAR["seed"], batch=SINGULAR["batch"], vocab=SINGULAR["vocab"])


def drafting_inputs():
    from bench import c4_workload

    p = DRAFTING
    return c4_workload(seed=p["seed"], rows=p["rows"], slots=p["slots"], gamma=p["gamma"],
                       draft_vocab=p["draft_vocab"], target_vocab=p["target_vocab"], timestep=p["timestep"])


def multistep_inputs():
    from bench import c3_workload

    return c3_workload(seed=MULTISTEP["seed"], batch=MULTISTEP["batch"], gamma=MULTISTEP["gamma"],
                       vocab=MULTISTEP["vocab"])


def topk_inputs():
    from bench import spiked_logits

    return spiked_logits(TOPK["rows"], TOPK["vocab"], TOPK["seed"], torch.float32)


def row_record(e) -> dict:
    return {"token": e.token, "greedy": e.greedy, "knife": e.knife, "logprob": e.logprob,
            "top_tokens": list(e.top_tokens), "top_logprobs": list(e.top_logprobs),
            "probs": None if e.probs is None else {str(k): v for k, v in sorted(e.probs.items())}}


def request_record(e) -> dict:
    return {"offset": e.offset, "tokens": list(e.tokens), "greedy": e.greedy, "knife": e.knife,
            "logprobs": list(e.logprobs), "top_tokens": [list(t) for t in e.top_tokens],
            "top_logprobs": [list(v) for v in e.top_logprobs],
            "row_indices": [[int(i) for i in idx] for idx in e.row_indices]}


def singular_case() -> dict:
    from oracle import sampler as oracle

    w = singular_inputs()
    state = oracle.State.from_buffers(w.buffers)
    expected = oracle.singular(w.logits, state, scope="target", logprobs=True, max_top_logprobs=5)

    return {"params": SINGULAR, "inputs": {"logits": digest(w.logits), **state_digests(w.buffers, "singular")},
            "rows": [row_record(e) for e in expected]}


def drafting_case() -> dict:
    from oracle import sampler as oracle

    w = drafting_inputs()
    state = oracle.State.from_buffers(w.buffers)
    expected = oracle.singular(w.logits, state, scope="draft", timestep=w.timestep,
                               slot_mapping=w.slot_mapping.tolist(), d2t=w.d2t, drafted=w.tokens,
                               history=w.timestep, probs=True, max_top_logprobs=5)
    inputs = {"logits": digest(w.logits), "d2t": digest(w.d2t), "slot_mapping": digest(w.slot_mapping),
              "tokens": digest(w.tokens), **state_digests(w.buffers, "drafting")}

    return {"params": DRAFTING, "inputs": inputs, "rows": [row_record(e) for e in expected]}


def multistep_case() -> dict:
    from oracle import sampler as oracle

    w = multistep_inputs()
    state = oracle.State.from_buffers(w.buffers)
    expected = oracle.multistep(w.logits, state, w.drafted, w.cu_seqlens, probabilities=w.probabilities,
                                logprobs=True, max_top_logprobs=20)
    inputs = {"logits": digest(w.logits), "drafted": digest(w.drafted),
              "probabilities": digest(w.probabilities), **state_digests(w.buffers, "multistep")}

    return {"params": MULTISTEP, "cu_seqlens": list(w.cu_seqlens), "inputs": inputs,
            "requests": [request_record(e) for e in expected]}


def topk_case() -> dict:
    from oracle.topk import topk

    x = topk_inputs()
    values, indices = topk(x, TOPK["k"])

    return {"params": TOPK, "inputs": {"logits": digest(x)},
            "values": [[float(v) for v in row] for row in values],
            "indices": [[int(i) for i in row] for row in indices]}


CASES = {"singular": singular_case, "drafting": drafting_case, "multistep": multistep_case, "topk": topk_case}

# Tensors of a case's workload besides the logits and its SamplingBuffers
EXTRA = {"singular": (), "drafting": ("d2t", "slot_mapping", "tokens"),
         "multistep": ("drafted", "probabilities"), "topk": ()}


def workload_tensors(name: str, w) -> dict:
    """Every tensor of a case's workload by attribute path (plain tensors, CPU)."""

    import dataclasses

    from sonic_sampler.core.flags import Flags

    if name == "topk":

        return {"logits": w}

    out = {"logits": w.logits}

    for attr in EXTRA[name]:

        out[attr] = getattr(w, attr)

    def walk(obj, path):

        if isinstance(obj, Flags):

            out[path + ".packed"] = obj.packed

        elif dataclasses.is_dataclass(obj):

            for f in dataclasses.fields(obj):

                walk(getattr(obj, f.name), f"{path}.{f.name}")

        elif isinstance(obj, torch.Tensor):

            out[path] = obj

    walk(w.buffers, "buffers")

    return {k: torch.Tensor.as_subclass(v, torch.Tensor).detach().clone() for k, v in out.items()}


def fixture_inputs(name: str):
    """The case's workload with the exact input bits the fixture was made from.

    torch's vectorized CPU samplers (normal, exponential) give different low bits on different
    vector units, so the generator runs in a child process under the fixtures' settings and the
    tensors it produced are copied into a workload built here (same structure)."""

    import subprocess
    import tempfile

    with tempfile.TemporaryDirectory() as tmp:

        path = Path(tmp) / f"{name}.pt"
        env = dict(os.environ, ATEN_CPU_CAPABILITY="default", OMP_NUM_THREADS="1")
        out = subprocess.run([sys.executable, str(Path(__file__).resolve()), "--inputs", name, "--out", str(path)],
                             env=env, capture_output=True, text=True, timeout=300)

        if out.returncode != 0:

            raise RuntimeError(f"generating the {name} fixture inputs failed:\n{out.stdout}{out.stderr}")

        saved = torch.load(path, weights_only=True)

    w = globals()[f"{name}_inputs"]()
    here = workload_tensors(name, w)

    if saved.keys() != here.keys():

        raise RuntimeError(f"{name}: the workload's tensors differ from the generated ones")

    if name == "topk":

        return saved["logits"]

    def target(path):

        obj = w

        for part in path.split("."):

            obj = getattr(obj, part)

        return obj

    for key, tensor in saved.items():

        target(key).copy_(tensor)

    return w


def main(argv=None) -> int:
    import argparse

    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--out", type=Path, default=HERE,
                        help="folder the fixtures are written to (with --inputs: the tensor file)")
    parser.add_argument("--inputs", choices=sorted(CASES), default=None,
                        help="write only this case's input tensors (a torch file of plain tensors) to --out")
    args = parser.parse_args(argv)
    torch.set_num_threads(1)

    if args.inputs:

        name = args.inputs
        w = globals()[f"{name}_inputs"]()
        torch.save(workload_tensors(name, w), args.out)

        return 0

    args.out.mkdir(parents=True, exist_ok=True)

    for name, make in CASES.items():

        case = make()
        case["torch"] = torch.__version__
        path = args.out / f"{name}.json"
        path.write_text(json.dumps(case, indent=None, separators=(",", ":")) + "\n")
        print(f"wrote {path} ({path.stat().st_size} bytes)")

    return 0


if __name__ == "__main__":
    sys.exit(main())
