"""GPU parity: block-aligned permutation against the C oracle and the numpy restatement."""
import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle.moe_oracle import moe_align_block_size_np

pytestmark = pytest.mark.gpu


def gen_ids(kind, T, k, E, seed):
    rng = np.random.default_rng(seed)
    if kind == "uniform":
        return np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    if kind == "zipf":
        p = 1.0 / np.arange(1, E + 1) ** 1.2
        p = p[rng.permutation(E)]
        p /= p.sum()
        return np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)]).astype(
            np.int32)
    if kind == "half_empty":
        return np.stack([rng.permutation(E // 2)[:k] for _ in range(T)]).astype(np.int32)
    if kind == "remote":
        ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
        return np.where(ids >= E // 2, -1, ids).astype(np.int32)
    if kind == "repeat":  # same expert in several slots (allowed by the align contract)
        return rng.integers(0, 3, size=(T, k)).astype(np.int32)
    raise ValueError(kind)


CASES = [(1, 8, 128, 16), (8, 8, 128, 16), (64, 8, 128, 16), (256, 8, 128, 64),
         (1000, 8, 128, 64), (1024, 8, 128, 64), (1025, 8, 128, 64), (2048, 8, 128, 64),
         (8192, 8, 128, 64), (64, 2, 8, 16), (3, 2, 3, 4), (4097, 3, 512, 128),
         (100, 4, 16, 512), (2000, 8, 64, 256)]


@pytest.mark.parametrize("T,k,E,bm", CASES)
@pytest.mark.parametrize("kind", ["uniform", "zipf", "half_empty", "remote", "repeat"])
def test_align_bitexact(dev, tsm, T, k, E, bm, kind):
    if kind in ("uniform", "zipf", "half_empty", "remote") and k > E // 2:
        pytest.skip("k larger than the experts available to this distribution")
    print(f"align T={T} k={k} E={E} bm={bm} {kind}", flush=True)
    ids = gen_ids(kind, T, k, E, seed=T + E)
    s, e, t = tsm.moe_align_block_size(torch.from_numpy(ids).to(dev), bm, E)
    os_, oe, ot = c_oracle.align(ids, bm, E)
    ns, ne, nt = moe_align_block_size_np(ids, bm, E)
    assert np.array_equal(os_, ns) and np.array_equal(oe, ne) and np.array_equal(ot, nt)
    assert np.array_equal(s.cpu().numpy(), os_)
    assert np.array_equal(e.cpu().numpy(), oe)
    assert np.array_equal(t.cpu().numpy(), ot)


def test_align_docstring_example(dev, tsm):
    """tinykernels.py:1075-1098."""
    s, e, t = tsm.moe_align_block_size(torch.tensor([[1, 0], [1, 2]], device=dev), 4, 3)
    assert s.cpu().tolist() == [1, 4, 4, 4, 0, 2, 4, 4, 3, 4, 4, 4, 4, 4, 4, 4]
    assert e.cpu().tolist() == [0, 1, 2, -1]
    assert t.cpu().tolist() == [12]


def test_align_int64_ids_and_empty(dev, tsm):
    ids = torch.tensor([[5, -1, 2]], dtype=torch.int64, device=dev)
    s, e, t = tsm.moe_align_block_size(ids, 2, 6)
    os_, oe, ot = c_oracle.align(ids.cpu().numpy(), 2, 6)
    assert np.array_equal(s.cpu().numpy(), os_) and np.array_equal(e.cpu().numpy(), oe)
    empty = torch.empty(0, 8, dtype=torch.int32, device=dev)
    s, e, t = tsm.moe_align_block_size(empty, 16, 128)
    os_, oe, ot = c_oracle.align(np.empty((0, 8), np.int32), 16, 128)
    assert np.array_equal(s.cpu().numpy(), os_) and np.array_equal(e.cpu().numpy(), oe)
    assert int(t.item()) == 0
