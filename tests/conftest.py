import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_addoption(parser):
    parser.addoption("--emulate", action="store_true",
                     help="run the -m gpu tests on the CPU build of the kernels (tests/emu): a "
                          "pre-flight check of kernels and tests at small sizes, not GPU parity")


@pytest.fixture(scope="session")
def _emulation(request):
    if not request.config.getoption("--emulate"):
        yield False
        return
    sys.path.insert(0, os.path.join(ROOT, "tests", "emu"))
    import harness
    with harness.emulated(asan=os.environ.get("TSM_EMU_ASAN") == "1"):
        yield True


@pytest.fixture(scope="session")
def dev(_emulation):
    import torch
    if _emulation:
        return torch.device("cpu")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def tsm(_emulation):
    import tinyserve_amd
    return tinyserve_amd


@pytest.fixture(scope="session")
def qwen_layer(dev):
    """Qwen3-30B-A3B-shaped layer weights (H=2048, E=128, I=768), bf16, drawn on the GPU, seed 0.
    Returns (gate_w, w13, w2) on the GPU and the same tensors on the CPU for the oracle."""
    import torch
    from oracle.moe_oracle import make_layer
    _, gate_w, w13, w2 = make_layer(1, 2048, 128, 768, torch.bfloat16, seed=0, device=dev)
    return (gate_w, w13, w2), (gate_w.cpu(), w13.cpu(), w2.cpu())
