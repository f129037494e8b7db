"""Shared test plumbing.

* registers the ``gpu`` marker (tests that launch HIP kernels on an MI355X);
* builds the HIP library / CPU oracle when nothing is built yet;
* converts between torch bf16 tensors and the oracle's uint16 bit arrays;
* ``assert_bf16_close``: the parity bar for bf16 outputs - at most ``max_ulp``
  bf16 ulps from the oracle and within atol/rtol 1e-2 (the bf16 tolerance the
  benchmark definition in BASELINE.json states).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import build as oracle_build  # noqa: E402
from oracle import oracle as O  # noqa: E402
from starter_amd import build as hip_build  # noqa: E402

ATOL = 1e-2
RTOL = 1e-2


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs HIP kernels)")


def pytest_sessionstart(session):
    if not oracle_build.LIBRARY.exists():
        oracle_build.build()
    if not hip_build.LIBRARY.exists():
        hip_build.build()


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> uint16 numpy bit array of the same shape."""
    assert t.dtype == torch.bfloat16
    return t.detach().cpu().contiguous().view(torch.uint16).numpy()


def tensor(b: np.ndarray, device="cpu") -> torch.Tensor:
    """uint16 bit array -> bf16 tensor on ``device``."""
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint16)).view(torch.bfloat16).to(device)


def gen(seed: int = 0) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def normal(shape, mean=0.0, std=1.0, g=None) -> torch.Tensor:
    """f32 draws N(mean, std) on a CPU generator, rounded to bf16 (the input
    recipe of the BASELINE.json configurations)."""
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std + mean).to(torch.bfloat16)


def assert_bf16_close(actual, expected, max_ulp: int = 1, atol: float = ATOL, rtol: float = RTOL,
                      min_exact: float | None = None, what: str = ""):
    """actual/expected: bf16 tensors or uint16 bit arrays of equal shape."""
    a = bits(actual) if isinstance(actual, torch.Tensor) else np.asarray(actual, dtype=np.uint16)
    e = bits(expected) if isinstance(expected, torch.Tensor) else np.asarray(expected, dtype=np.uint16)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    if a.size == 0:
        return
    av, ev = O.bf16_value(a), O.bf16_value(e)
    nan_a, nan_e = np.isnan(av), np.isnan(ev)
    assert np.array_equal(nan_a, nan_e), f"{what}: NaN positions differ"
    ok = ~nan_a
    ulp = O.ulp_distance(a[ok], e[ok])
    worst = int(ulp.max()) if ulp.size else 0
    assert worst <= max_ulp, f"{what}: max {worst} bf16 ulp > {max_ulp} ({int((ulp > max_ulp).sum())} elements)"
    np.testing.assert_allclose(av[ok], ev[ok], atol=atol, rtol=rtol, err_msg=what)
    if min_exact is not None and ulp.size:
        exact = float((ulp == 0).mean())
        assert exact >= min_exact, f"{what}: only {exact:.5f} bit-exact (< {min_exact})"


def assert_bits_exact(actual, expected, what: str = ""):
    """Bit-for-bit equality of two bf16 results (NaNs compared as NaN-ness,
    since NaN payloads are not part of any contract)."""
    a = bits(actual) if isinstance(actual, torch.Tensor) else np.asarray(actual, dtype=np.uint16)
    e = bits(expected) if isinstance(expected, torch.Tensor) else np.asarray(expected, dtype=np.uint16)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    nan_a, nan_e = np.isnan(O.bf16_value(a)), np.isnan(O.bf16_value(e))
    assert np.array_equal(nan_a, nan_e), f"{what}: NaN positions differ"
    diff = (a != e) & ~nan_a
    assert not diff.any(), (f"{what}: {int(diff.sum())} of {a.size} elements differ, max "
                            f"{int(O.ulp_distance(a[diff], e[diff]).max())} bf16 ulp")


GOLDEN = Path(__file__).with_name("golden") / "golden.npz"


@pytest.fixture(scope="session")
def golden() -> dict:
    """tests/golden/golden.npz grouped by case: {case: {name: array}}."""
    groups: dict = {}
    with np.load(GOLDEN, allow_pickle=False) as data:
        for key in data.files:
            case, _, name = key.partition("/")
            groups.setdefault(case, {})[name] = data[key]
    return groups
