import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "emu_tokens(n): a GPU test whose batch is n tokens (for "
                                       "--emulate-max-tokens when the size is not a T parameter)")
    config.addinivalue_line("markers", "emu_skip(reason): a GPU test the CPU emulation cannot run")


def pytest_addoption(parser):
    parser.addoption("--emulate", action="store_true",
                     help="run the -m gpu tests on the CPU build of the kernels (tests/emu): a "
                          "pre-flight check of kernels and tests at small sizes, not GPU parity")
    parser.addoption("--emulate-max-tokens", type=int, default=1024,
                     help="with --emulate, skip cases of more tokens than this (a Qwen3-30B "
                          "layer of 512 tokens takes about 80 s on the emulation)")


# A GPU test that has not finished in this long is hung (the largest take seconds): the thread
# method of pytest-timeout dumps every stack, naming the test, and ends the process instead of
# leaving it to the job's own time limit.
GPU_TEST_TIMEOUT_S = 300


def pytest_collection_modifyitems(config, items):
    if not config.getoption("--emulate"):
        for item in items:
            if item.get_closest_marker("gpu") and not item.get_closest_marker("timeout"):
                item.add_marker(pytest.mark.timeout(GPU_TEST_TIMEOUT_S, method="thread"))
        return
    limit = config.getoption("--emulate-max-tokens")
    for item in items:
        why = item.get_closest_marker("emu_skip")
        if why is not None:
            item.add_marker(pytest.mark.skip(reason=f"not on the CPU emulation: {why.args[0]}"))
            continue
        mark = item.get_closest_marker("emu_tokens")
        callspec = getattr(item, "callspec", None)
        T = mark.args[0] if mark else (callspec.params.get("T") if callspec else None)
        if isinstance(T, int) and T > limit:
            item.add_marker(pytest.mark.skip(
                reason=f"{T} tokens: above --emulate-max-tokens={limit}"))


@pytest.fixture(scope="session")
def _emulation(request):
    if not request.config.getoption("--emulate"):
        yield False
        return
    sys.path.insert(0, os.path.join(ROOT, "tests", "emu"))
    import harness
    with harness.emulated(harness.sanitizer_from_env()):
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
