"""The GPU parity suite again, with every library workspace poisoned.

Every scratch buffer the Python layer hands to the library is filled with
0xFF bytes (NaN as floats, -1 as integers, the highest key as 64-bit keys)
instead of being left as the allocator returns it, usually zeros or
finite leftovers.  A kernel that reads scratch it did not write then shows
up as a parity failure, even when the value only meets a zero weight:
0 * NaN is NaN.  Each test of tests/test_gpu_parity.py is collected here a
second time and runs under the poisoned allocator.
"""
import pytest
import torch

from tests.test_gpu_parity import *  # noqa: F401,F403  (re-collects every parity test)

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _poisoned_workspace(monkeypatch):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from strict_topk import _lib
    _lib.lib()   # fail loudly if the HIP library is missing
    monkeypatch.setattr(_lib, "workspace", lambda nbytes, device: torch.full(
        (max(int(nbytes), 1),), 255, dtype=torch.uint8, device=device))
