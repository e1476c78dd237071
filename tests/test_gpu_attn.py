"""GPU parity of the attention-side kernels (csrc/attn.hip) against the oracle restatement of
serve.py's RMSNorm / rotary / torch_ref_attention (oracle/attn_oracle.py).

Tolerances: q/k norm + RoPE within one bf16 ulp of the oracle (the kernel's reciprocal square
root differs from torch's); attention outputs within 8e-3 + 2^-7 |ref| (outputs are convex
combinations of V rows of magnitude ~1, the probabilities enter the P.V product in bf16 as in
the reference's Triton kernel, and the output itself is rounded to bf16: half an ulp of a value
near 2 is already 2^-8); argmax exact."""

import pytest
import torch

from oracle.attn_oracle import paged_attention_ref, qk_norm_rope_ref

pytestmark = pytest.mark.gpu


def attn_close(out, ref, what=""):
    out, ref = out.float().cpu(), ref.float().cpu()
    assert torch.isfinite(out).all(), what
    err = (out - ref).abs()
    bound = 8e-3 + ref.abs() * 2.0 ** -7
    print(f"  {what} max abs err {err.max().item():.3e}", flush=True)
    assert bool((err <= bound).all()), (what, float((err / bound).max()))


def ulp_close(out, ref):
    out, ref = out.double().cpu(), ref.double().cpu()
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -126))) - 7)
    bad = (out - ref).abs() > ulp
    assert not bool(bad.any()), f"{int(bad.sum())} elements beyond 1 bf16 ulp"


def build_batch(dev, q_lens, kv_lens, H, Hkv, D, page, seed, nan_tail=True):
    """Random paged K/V for each request's context (distinct random pages, page 0 unused),
    NaN in the unused slots of each last page, and the packed queries."""
    from tinyserve_amd.attention import PagedKVCache
    g = torch.Generator().manual_seed(seed)
    need = sum(-(-n // page) for n in kv_lens) + 1
    num_pages = need + 7
    kc = torch.randn(num_pages, page, Hkv, D, generator=g).bfloat16()
    vc = torch.randn(num_pages, page, Hkv, D, generator=g).bfloat16()
    perm = (torch.randperm(num_pages - 1, generator=g) + 1).tolist()
    maxp = max(1, max(-(-n // page) for n in kv_lens))
    bt = torch.zeros(len(kv_lens), maxp + 2, dtype=torch.int32)
    for b, n in enumerate(kv_lens):
        for j in range(-(-n // page)):
            bt[b, j] = perm.pop()
        if nan_tail and n % page:
            last = int(bt[b, (n - 1) // page])
            kc[last, n % page:] = float("nan")
            vc[last, n % page:] = float("nan")
    qsl = [0]
    for n in q_lens:
        qsl.append(qsl[-1] + n)
    q = torch.randn(qsl[-1], H, D, generator=g).bfloat16()
    cache = PagedKVCache(kc.to(dev), vc.permute(0, 2, 3, 1).contiguous().to(dev))
    return q, kc, vc, cache, bt, qsl


class Meta:
    def __init__(self, dev, qsl, kv_lens, bt):
        cu = [0]
        for n in kv_lens:
            cu.append(cu[-1] + n)
        self.query_start_loc = torch.tensor(qsl, dtype=torch.int32, device=dev)
        self.cu_seqlens_k = torch.tensor(cu, dtype=torch.int32, device=dev)
        self.block_table = bt.to(dev)
        self.num_seqs = len(kv_lens)
        self.max_query_len = max(qsl[i + 1] - qsl[i] for i in range(len(kv_lens)))


CASES = [
    # (H, Hkv, D, page, q_lens, kv_lens): Qwen3-30B heads (group 8, D 128), smaller groups
    (32, 4, 128, 16, [1, 1, 1, 1], [1, 33, 300, 64]),                 # decode only
    (32, 4, 128, 16, [512, 1, 37, 0, 5], [512, 700, 90, 0, 5]),        # mixed, chunked prefill
    (8, 4, 64, 8, [3, 1, 17, 2], [9, 129, 17, 2]),                     # group 2, D 64
    (16, 16, 64, 4, [40, 1], [40, 1]),                                 # group 1, page 4
    (16, 1, 128, 32, [7, 1], [100, 1000]),                             # group 16
]


@pytest.mark.parametrize("H,Hkv,D,page,q_lens,kv_lens", CASES)
def test_paged_attention_against_oracle(dev, H, Hkv, D, page, q_lens, kv_lens):
    from tinyserve_amd.attention import paged_attention
    print(f"attention H={H} Hkv={Hkv} D={D} page={page} q={q_lens} kv={kv_lens}", flush=True)
    q, kc, vc, cache, bt, qsl = build_batch(dev, q_lens, kv_lens, H, Hkv, D, page, seed=H + D)
    meta = Meta(dev, qsl, kv_lens, bt)
    out = paged_attention(q.to(dev), cache.k, cache.v, meta, D ** -0.5)
    ref = paged_attention_ref(q.float(), kc.float(), vc.float(), qsl, kv_lens, bt, D ** -0.5)
    attn_close(out, ref, "paged attention")


# split-KV decode: (H, Hkv, D, page, q_lens, kv_lens, num_splits); 33 keys over 16 splits leaves
# most splits empty, the mixed batch keeps its prefill request on the unsplit launch
SPLIT_CASES = [
    (32, 4, 128, 16, [1], [4000], 16),
    (32, 4, 128, 16, [1, 1, 1], [33, 1000, 1], 16),
    (8, 4, 64, 8, [1, 1, 5, 1], [700, 1, 300, 2049], 4),
    (16, 1, 128, 32, [1, 1], [257, 64], 2),
]


@pytest.mark.parametrize("H,Hkv,D,page,q_lens,kv_lens,splits", SPLIT_CASES)
def test_split_kv_decode_against_oracle(dev, H, Hkv, D, page, q_lens, kv_lens, splits):
    from tinyserve_amd.attention import paged_attention
    print(f"split-KV H={H} Hkv={Hkv} D={D} q={q_lens} kv={kv_lens} splits={splits}", flush=True)
    q, kc, vc, cache, bt, qsl = build_batch(dev, q_lens, kv_lens, H, Hkv, D, page, seed=splits)
    meta = Meta(dev, qsl, kv_lens, bt)
    ref = paged_attention_ref(q.float(), kc.float(), vc.float(), qsl, kv_lens, bt, D ** -0.5)
    out = paged_attention(q.to(dev), cache.k, cache.v, meta, D ** -0.5, num_splits=splits)
    attn_close(out, ref, f"{splits} splits")
    # the automatic choice from max_seq_len (a small batch of long contexts splits)
    meta.max_seq_len = max(kv_lens)
    attn_close(paged_attention(q.to(dev), cache.k, cache.v, meta, D ** -0.5), ref, "auto")


@pytest.mark.emu_skip("HIP graph capture")
def test_paged_attention_graph_replay(dev):
    """A decode step's attention captured in a HIP graph replays with new lengths and pages
    (the grid depends only on T, num_seqs and Hkv)."""
    from tinyserve_amd.attention import paged_attention
    H, Hkv, D, page = 32, 4, 128, 16
    q, kc, vc, cache, bt, qsl = build_batch(dev, [1] * 4, [50, 200, 17, 400], H, Hkv, D, page,
                                            seed=5, nan_tail=False)
    meta = Meta(dev, qsl, [50, 200, 17, 400], bt)
    qd = q.to(dev)
    eager = paged_attention(qd, cache.k, cache.v, meta, D ** -0.5)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        paged_attention(qd, cache.k, cache.v, meta, D ** -0.5)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = paged_attention(qd, cache.k, cache.v, meta, D ** -0.5)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    # shorter contexts in place: the replay follows the device metadata
    kv2 = [49, 3, 17, 250]
    cu = torch.tensor([0, 49, 52, 69, 319], dtype=torch.int32, device=dev)
    meta.cu_seqlens_k.copy_(cu)
    graph.replay()
    torch.cuda.synchronize()
    ref = paged_attention_ref(q.float(), kc.float(), vc.float(), qsl, kv2, bt, D ** -0.5)
    attn_close(out, ref, "replay with shorter contexts")


@pytest.mark.parametrize("T,H,Hkv,D", [(5, 32, 4, 128), (300, 8, 2, 64), (1, 4, 4, 128)])
@pytest.mark.parametrize("norm", [True, False])
def test_qk_norm_rope_and_cache_write(dev, T, H, Hkv, D, norm):
    from tinyserve_amd.attention import PagedKVCache, qk_norm_rope
    print(f"qk_norm_rope T={T} H={H} Hkv={Hkv} D={D} norm={norm}", flush=True)
    g = torch.Generator().manual_seed(T * H + D)
    qkv = (torch.randn(T, (H + 2 * Hkv) * D, generator=g) * 3).bfloat16()
    pos = torch.randint(0, 4096, (T,), generator=g).double()
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = pos[:, None] * inv[None, :]
    cos, sin = ang.cos().float(), ang.sin().float()
    qw = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16() if norm else None
    kw = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16() if norm else None
    q, k, v = qkv.split([H * D, Hkv * D, Hkv * D], dim=-1)
    q, k, v = q.reshape(T, H, D), k.reshape(T, Hkv, D), v.reshape(T, Hkv, D)
    rq, rk = qk_norm_rope_ref(q, k, cos, sin, qw, kw, 1e-6)
    page = 16
    cache = PagedKVCache.allocate(T // page + 3, page, Hkv, D, dev)
    slots = torch.randperm((T // page + 2) * page, generator=g)[:T] + page  # page 0 unused
    slots[0] = -1                                                         # a token not written
    d_qkv = qkv.to(dev)
    dq, dk, dv = d_qkv.split([H * D, Hkv * D, Hkv * D], dim=-1)
    dq, dk, dv = dq.view(T, H, D), dk.view(T, Hkv, D), dv.view(T, Hkv, D)   # strided views
    qk_norm_rope(dq, dk, cos.to(dev), sin.to(dev), None if qw is None else qw.to(dev),
                 None if kw is None else kw.to(dev), 1e-6, dv, cache.k, cache.v, slots.to(dev))
    ulp_close(dq, rq)
    ulp_close(dk, rk)
    assert torch.equal(dv.cpu(), v)   # v itself is left alone
    kcache, vcache = cache.k.cpu(), cache.v.cpu()
    for t in range(T):
        sl = int(slots[t])
        if sl < 0:
            continue
        assert torch.equal(kcache[sl // page, sl % page], dk[t].cpu())
        assert torch.equal(vcache[sl // page, :, :, sl % page], v[t])
    assert bool((kcache[0] == 0).all()) and bool((vcache[0] == 0).all())


def test_greedy_argmax(dev):
    from tinyserve_amd.attention import greedy_argmax
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 151936, generator=g)
    x[3, 100] = x[3, 5000] = 50.0          # tie: the lower index
    x[4] = -float("inf")
    x[4, 77] = -1e30
    for dt in (torch.float32, torch.bfloat16):
        xd = x.to(dt)
        got = greedy_argmax(xd.to(dev)).cpu()
        assert torch.equal(got, xd.float().argmax(-1)), dt
    assert int(greedy_argmax(x.to(dev))[3]) == 100
