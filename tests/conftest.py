import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libdeltaattn.so")


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; GPU tests fail loudly when the native library is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from deltaattention_amd import _native
    _native.lib()  # raises NativeLibraryError if libdeltaattn.so is not built
    return torch.device("cuda:0")


def announce(msg: str) -> None:
    """Name the case before a GPU step, so a fault that ends the process is attributable."""
    print(f"[case] {msg}", flush=True)


def oracle_arith(keys) -> str:
    """The oracle's name for the product's default selection arithmetic on these keys:
    "native" evaluates the Euclidean distance in the keys' own type (tritonModules.py:
    55-58), which the oracle calls "bf16", "fp16" or (fp32 keys) "fp32"."""
    import torch
    return {torch.float16: "fp16", torch.float32: "fp32"}.get(keys.dtype, "bf16")
