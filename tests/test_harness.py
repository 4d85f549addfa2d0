"""The parity criterion of the library self-tests: correct output passes, planted bugs fail.
Restates the expectations of the reference's tests/test_tools.py:38-78 on CPU tensors."""
import math

import torch

from _harness import compare, significance


def _noisy(r, rel, seed):
    g = torch.Generator().manual_seed(seed)
    return r + rel * r.abs().mean() * torch.randn(r.shape, generator=g)


def _ref(shape, seed=0):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed))


def test_compare_accepts_same_noise_level():
    r = _ref((64, 1024))
    assert compare([r], [_noisy(r, 1e-2, 1)], [_noisy(r, 1e-2, 2)])["pass"]


def test_compare_catches_localized_bug_by_rows():
    r = _ref((64, 1024))
    c = _noisy(r, 1e-2, 2)
    c[5] *= 1.05  # one row off by 5%: hardly moves the tensor-wide numbers
    res = compare([r], [_noisy(r, 1e-2, 1)], [c])
    out = res["outputs"][0]
    assert not res["pass"] and out["bad_rows"] == 1 and out["worst_row"]["row"] == 5


def test_compare_catches_nonfinite_and_shape():
    r = _ref((8, 128))
    c = r.clone()
    c[0, 0] = float("nan")
    res = compare([r], [r], [c])
    assert not res["pass"] and res["outputs"][0]["nonfinite"] == 1
    assert not compare([r], [r], [r[:4]])["pass"]
    assert not compare([r, r], [r, r], [r])["pass"]


def test_compare_catches_global_scale_error():
    r = _ref((32, 256))
    assert not compare([r], [_noisy(r, 1e-3, 1)], [r * 1.01])["pass"]


def test_compare_slack_is_relative_to_original():
    r = _ref((32, 256))
    orig = _noisy(r, 1e-2, 1)
    assert compare([r], [orig], [_noisy(r, 1.8e-2, 3)])["pass"]       # within 2x the original
    assert not compare([r], [orig], [_noisy(r, 4e-2, 3)])["pass"]     # 4x the original's error


def test_compare_integer_outputs_exact():
    a = torch.arange(10)
    assert compare([a], [a], [a.clone()])["pass"]
    assert not compare([a], [a], [a + 1])["pass"]


def test_compare_reports_worst_and_where():
    r = _ref((16, 64))
    c = r.clone()
    c[3, 7] += 10.0
    res = compare([r], [r], [c])
    w = res["outputs"][0]["worst"]
    assert not res["pass"] and w["index"] == [3, 7] and math.isclose(w["got"] - w["ref"], 10.0, rel_tol=1e-5)


def test_significance():
    assert significance({"rounds": [10, 11]}, {"rounds": [5, 6]}) == "faster"
    assert significance({"rounds": [10, 11]}, {"rounds": [10.5, 12]}) == "within noise"
    assert significance({"rounds": [5, 6]}, {"rounds": [10, 11]}) == "slower"
