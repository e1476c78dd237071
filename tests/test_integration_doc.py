"""The ctypes binding shown in INTEGRATION.md loads the library and marshals its arguments as
written (no GPU needed: an empty batch returns before any launch, and an invalid argument comes
back as a status code with its message)."""
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def binding_source():
    """The python block of INTEGRATION.md's reference-side binding, with the library path set to
    the in-tree build."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    section = text.split("## Reference-side binding", 1)[1]
    code = re.search(r"```python\n(.*?)```", section, re.S).group(1)
    lib = os.path.join(ROOT, "tinyserve_amd", "libtinyserve_moe.so")
    assert 'ctypes.CDLL("libtinyserve_moe.so")' in code
    return code.replace('ctypes.CDLL("libtinyserve_moe.so")', f"ctypes.CDLL({lib!r})")


def test_documented_binding_marshals(monkeypatch):
    if not os.path.exists(os.path.join(ROOT, "tinyserve_amd", "libtinyserve_moe.so")):
        pytest.skip("library not built")
    ns = {}
    exec(compile(binding_source(), "INTEGRATION.md", "exec"), ns)

    class _Stream:
        cuda_stream = 0
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a, **k: _Stream())
    w, ids = ns["moe_route"](torch.empty(0, 128), 8, True, None)
    assert w.shape == (0, 8) and ids.shape == (0, 8)
    with pytest.raises(AssertionError, match="top_k"):
        ns["moe_route"](torch.empty(0, 128), 0, True, None)
