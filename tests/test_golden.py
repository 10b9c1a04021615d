"""The committed golden fixtures (tests/golden/*.json) against the oracle and the generators.

The oracle, rerun in a fresh process under the fixtures' settings (``ATEN_CPU_CAPABILITY=default``,
one thread), must write every fixture again byte for byte, so a change to the oracle's arithmetic
or to the generators shows here. The top-k fixture is also checked against a plain Python sort,
independent of torch.
"""

import json
import os
import subprocess
import sys

from pathlib import Path

import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = ("singular", "drafting", "multistep", "topk")


def load(name):

    return json.loads((GOLDEN / f"{name}.json").read_text())


def test_oracle_rewrites_every_fixture(tmp_path):

    env = dict(os.environ, ATEN_CPU_CAPABILITY="default", OMP_NUM_THREADS="1")
    out = subprocess.run([sys.executable, str(GOLDEN / "make_fixtures.py"), "--out", str(tmp_path)],
                         env=env, capture_output=True, text=True, timeout=600)

    assert out.returncode == 0, out.stdout + out.stderr

    for name in CASES:

        assert (tmp_path / f"{name}.json").read_bytes() == (GOLDEN / f"{name}.json").read_bytes(), name


@pytest.mark.parametrize("name", CASES)
def test_generators_reproduce_the_fixture_inputs(name):
    """The case's generator, run under the fixtures' settings, gives exactly the digested inputs."""

    from golden import make_fixtures as mf

    case = load(name)
    w = mf.fixture_inputs(name)

    if name == "topk":

        got = {"logits": mf.digest(w)}

    else:

        got = {"logits": mf.digest(w.logits), **mf.state_digests(w.buffers, name)}
        got.update({attr: mf.digest(getattr(w, attr)) for attr in mf.EXTRA[name]})

    assert got == case["inputs"]


def test_topk_fixture_is_the_stable_descending_order():
    """Every fixture row's indices are the first k of the columns sorted by (value desc, index asc)
    in plain Python, and its values are the row's values there."""

    from golden import make_fixtures as mf

    case = load("topk")
    x = mf.fixture_inputs("topk")
    k = case["params"]["k"]

    for r, row in enumerate(x.tolist()):

        order = sorted(range(len(row)), key=lambda c: (-row[c], c))[:k]

        assert case["indices"][r] == order
        assert case["values"][r] == [row[c] for c in order]


def test_fixtures_hold_sane_outputs():
    """Invariants of the stored outputs: emitted spans are drafts then one more token, offsets
    within each request's lookahead, logprobs <= 0, top logprobs in descending order."""

    multistep = load("multistep")
    cu = multistep["cu_seqlens"]

    for b, req in enumerate(multistep["requests"]):

        assert 0 <= req["offset"] <= cu[b + 1] - cu[b] - 1
        assert len(req["tokens"]) == req["offset"] + 1
        assert all(v <= 0.0 for v in req["logprobs"])

        for values in req["top_logprobs"]:

            assert values == sorted(values, reverse=True)

    for name in ("singular", "drafting"):

        for row in load(name)["rows"]:

            assert row["logprob"] is None or row["logprob"] <= 0.0
            assert row["top_logprobs"] == sorted(row["top_logprobs"], reverse=True)

            if row["probs"] is not None:

                assert abs(sum(row["probs"].values()) - 1.0) < 1e-3
