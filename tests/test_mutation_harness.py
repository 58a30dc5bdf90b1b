"""The mutation harness (tests/mutation/mutate.py) stays usable: every mutant still applies to the
current sources exactly once, and one planted kernel mistake, built and tested end to end, is
caught while the in-tree sources stay untouched. The full run (about 10 minutes) is
`python tests/mutation/mutate.py`; its last report is tests/mutation/results.txt."""
import hashlib
import importlib.util
import os
import sys

from conftest import ROOT

HARNESS = os.path.join(ROOT, "tests", "mutation", "mutate.py")


def load():
    if "kvb_mutate" in sys.modules:
        return sys.modules["kvb_mutate"]
    spec = importlib.util.spec_from_file_location("kvb_mutate", HARNESS)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["kvb_mutate"] = mod  # dataclasses look their module up by name
    spec.loader.exec_module(mod)
    return mod


def digest(rel):
    with open(os.path.join(ROOT, rel), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def test_every_mutant_applies_once():
    mut = load()
    assert mut.check_all() == []
    groups = {m.group for m in mut.MUTANTS}
    assert groups == set(mut.GROUP_TESTS)
    for g in groups:
        assert all(os.path.exists(os.path.join(ROOT, t)) for t in mut.GROUP_TESTS[g])


def test_a_planted_kernel_mistake_is_caught():
    mut = load()
    m = next(x for x in mut.MUTANTS if x.name == "block table ignored (logical = physical)")
    before = digest(m.path)
    status, summary = mut.run_one(m, fail_fast=True)
    assert status == "caught", summary
    assert digest(m.path) == before


def test_report_covers_every_mutant():
    mut = load()
    with open(os.path.join(ROOT, "tests", "mutation", "results.txt")) as f:
        report = f.read()
    for m in mut.MUTANTS:
        assert f"{m.name}: caught" in report, m.name
