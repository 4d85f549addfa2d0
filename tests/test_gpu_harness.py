"""The timing half of the harness on the GPU, restating the reference's planted-behaviour
tests (tests/test_tools.py:58-72): a callable that syncs with the host is timed eagerly
without breaking the process, and an A/B of variants uses one timing mode for all of them."""
import pytest
import torch

from _harness import time_ab, time_calls
from krsi_testutil import log

pytestmark = pytest.mark.gpu


def test_failed_capture_does_not_poison_the_process():
    log("harness: host-syncing callable timed eagerly")
    x = torch.randn(1 << 16, device="cuda")
    res = time_calls([lambda: (x * 2).sum().item()], reps=2)
    assert res["mode"] == "eager" and "host sync" in res.get("note", "")
    torch.randn(8, device="cuda")  # the process still launches work normally
    y = torch.ones(1 << 10, device="cuda")
    assert time_calls([lambda: y * 2], reps=2)["mode"] == "graph"


def test_time_ab_uses_one_mode_for_all_variants():
    log("harness: time_ab with one graphable and one syncing variant")
    x = torch.randn(1 << 20, device="cuda")
    res = time_ab({"graphable": [lambda: x * 2], "syncs": [lambda: (x * 2).sum().item()]}, rounds=2, reps=3)
    assert res["graphable"]["mode"] == res["syncs"]["mode"] == "eager"
    assert "could not be graph-captured" in res["graphable"]["note"] and "host sync" in res["graphable"]["note"]


def test_compiled_callable_is_timed_by_graph_replay():
    # A torch.compile'd callable synchronises while it compiles, on its first call only; the
    # harness probes for host syncs after one warm call, so the compiled callable is captured.
    log("harness: compiled callable timed by graph replay")
    x = torch.randn(1 << 16, device="cuda")
    f = torch.compile(lambda: x * 2 + 1)
    res = time_calls([f], reps=2)
    assert res["mode"] == "graph", res.get("note")
