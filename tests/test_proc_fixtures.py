"""The compiled Proc of whole programs against the reference's own compile
passes: tests/golden/proc_fixtures.json holds the listing the reference
prints for each program (written by tests/golden/make_proc_fixtures.py in
the build container, which imports the reference's passes); this front end
must print the same listing line for line -- node ids, fusion groups,
statement order, access expressions, arena sizes and tetris offsets.
Trailing spaces are not compared (the reference ends ``TEMP Alloc`` lines
with one)."""
import json
import pathlib
import sys

import pytest

GOLDEN = pathlib.Path(__file__).parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_proc_fixtures as programs  # noqa: E402

FIXTURES = json.loads((GOLDEN / "proc_fixtures.json").read_text())


def _lines(text):
    return [line.rstrip() for line in text.splitlines()]


@pytest.mark.parametrize("name", sorted(programs.PROGRAMS))
def test_listing_matches_the_reference(name):
    want = _lines(FIXTURES[name]["proc"])
    got = _lines(programs.our_listing(name))
    assert len(got) == len(want)
    for i, (g, w) in enumerate(zip(got, want)):
        assert g == w, f"{name} line {i + 1}"


@pytest.mark.parametrize("name,used,total", [("transformer_example", 2228, 4738), ("linear_example", 2040, 2040)])
def test_tetris_totals_match_the_reference(name, used, total):
    """The arena totals the reference printed for these programs
    (Success.png reports 2228 of 4738 floats for the 1-layer example)."""
    assert FIXTURES[name]["alloc"] == [f"ALLOC DEBUG: Using: {used} out of {total}"]
    first = _lines(FIXTURES[name]["proc"])[0]
    assert first.startswith("Alloc ") and first.endswith(f" {used}")
