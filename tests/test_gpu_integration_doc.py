"""The ctypes binding shown in INTEGRATION.md (the one a maintainer would add next to
tinykernels) runs as written against the in-tree library and matches the package's moe_route."""
import pytest
import torch
from test_integration_doc import binding_source as _binding_source

pytestmark = pytest.mark.gpu


@pytest.mark.emu_skip("the binding loads the GPU library and takes the current HIP stream")
@pytest.mark.parametrize("with_map", [False, True])
def test_documented_binding(dev, tsm, with_map):
    ns = {}
    exec(compile(_binding_source(), "INTEGRATION.md", "exec"), ns)
    g = torch.Generator().manual_seed(2)
    logits = torch.randn(33, 128, generator=g).to(dev)
    emap = None
    if with_map:
        emap = torch.arange(128, dtype=torch.int64)
        emap[100:] = -1
        emap = emap.to(dev)
    w, ids = ns["moe_route"](logits, 8, True, emap)
    w2, ids2 = tsm.moe_route(logits, 8, True, emap)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2) and torch.equal(w, w2)

