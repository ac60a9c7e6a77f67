"""Shared test setup. ``-m gpu`` tests run through ``libretrieve_amd.so`` on an MI355X and
compare with the CPU oracle (``oracle/``); ``-m "not gpu"`` tests cover the oracle against the
reference's golden vectors, the host logic and the C-ABI library's exports."""

from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X; runs the HIP library")


@pytest.fixture(scope="session")
def kat():
    arrays = dict(np.load(os.path.join(GOLDEN, "kat.npz")))
    with open(os.path.join(GOLDEN, "kat.json")) as f:
        meta = json.load(f)
    return arrays, meta


@pytest.fixture(scope="session")
def dev():
    """The GPU. A missing GPU or library is a failure, not a skip: these tests are the
    parity gate."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test without a GPU (run with -m 'not gpu' on CPU hosts)")
    import retrieve_amd.hip  # noqa: F401  (registers the ops; raises if the library is missing)

    return torch.device("cuda:0")


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))
