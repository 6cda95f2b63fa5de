"""Shared pytest setup: import paths, the `gpu` marker, seeded input helpers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "sts-web_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on cuda:0)")


@pytest.fixture(autouse=True)
def _gc_between_tests():
    """Cyclic garbage is collected between tests, never at an arbitrary point
    inside one: the library's handles free device memory when collected, and a
    free while a stream is being captured into a graph invalidates the capture."""
    import gc
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        gc.enable()
        gc.collect()


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0.  Fails (never skips) when no GPU is present."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a host without a GPU (run with -m 'not gpu')")
    import sts_attn
    sts_attn.load()
    return torch.device("cuda:0")


def scale_for(d: int) -> float:
    """head_dim^-0.5 in f32 (model.rs:705)."""
    return float(np.float32(d) ** np.float32(-0.5))
