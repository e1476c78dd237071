"""The qwen3_moe workload driver (tinyserve_amd/e2e.py) on a small shape, against the decoder
oracle (oracle/decoder_oracle.py, a restatement of serve.py's torch forward): prefill logits,
and greedy decoding teacher-forced through the oracle; plus determinism and graph replay.

Tolerance: logits within 3e-2 of the largest |logit| (bf16 activations through two layers; the
kernels and the oracle round at the same points but sum in different orders). A greedy token
must equal the oracle's argmax unless the oracle's top two logits are closer than that, or a
routing decision of that position was a near tie (k-th and (k+1)-th expert probabilities within
2e-3: the bf16 hidden states of the two computations differ by roundings, which may then pick
the other expert — legitimately, and with a visible effect on the logits)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def small_cfg():
    from tinyserve_amd.e2e import Qwen3MoeConfig
    return Qwen3MoeConfig(hidden_size=256, num_hidden_layers=2, num_attention_heads=4,
                          num_key_value_heads=2, head_dim=64, vocab_size=1000, num_experts=8,
                          num_experts_per_tok=2, moe_intermediate_size=512)


def reference_logits(model, ids, route_gaps=False):
    from oracle.decoder_oracle import decoder_reference
    sd = {n: t.detach().cpu() for n, t in model.state_dict().items()}
    return decoder_reference(sd, model.cfg, ids.cpu(), return_route_gaps=route_gaps)


def test_prefill_and_decode_against_oracle(dev):
    from tinyserve_amd.e2e import build_model, generate
    model = build_model(small_cfg(), device=dev, seed=3, router_logits="fp32")
    g = torch.Generator(device=dev).manual_seed(7)
    B, P, N = 4, 33, 6
    prompts = torch.randint(0, 1000, (B, P), device=dev, generator=g)
    toks, _, _ = generate(model, prompts, N, graph=True)
    full = torch.cat([prompts, toks[:, :-1]], 1)
    ref, gaps = reference_logits(model, full, True)     # [B, P + N - 1, vocab]
    steps = ref[:, P - 1:]                              # logits that chose each new token
    scale = steps.abs().max().item()
    top2 = steps.topk(2, dim=-1).values
    clear = ((top2[..., 0] - top2[..., 1]) > 3e-2 * scale) & (gaps[:, P - 1:] > 2e-3)
    agree = toks.cpu() == steps.argmax(-1)
    assert bool(agree[clear].all()), (toks.cpu(), steps.argmax(-1))
    assert clear.float().mean().item() > 0.5
    # prefill logits themselves (last prompt position) through the driver's forward
    from tinyserve_amd.e2e import PagedBatch
    batch = PagedBatch(B, P, 16, dev)
    caches = model.new_caches(batch.num_pages, 16)
    meta, pos, last = batch.prefill_meta([P] * B)
    seq = torch.repeat_interleave(torch.arange(B, device=dev), P)
    meta.slot_mapping = batch.slots(seq, pos)
    logits = model(prompts.reshape(-1), pos, meta, caches, last).cpu()
    ok = gaps[:, P - 1] > 2e-3
    err = (logits - ref[:, P - 1]).abs().amax(-1)[ok]
    assert bool(ok.any()) and float(err.max()) <= 3e-2 * scale, (err, scale)


def test_generation_is_deterministic_and_graph_matches_eager(dev):
    from tinyserve_amd.e2e import build_model, generate
    model = build_model(small_cfg(), device=dev, seed=5)
    g = torch.Generator(device=dev).manual_seed(9)
    prompts = torch.randint(0, 1000, (3, 20), device=dev, generator=g)
    t1, _, _ = generate(model, prompts, 6, graph=True)
    t2, _, _ = generate(model, prompts, 6, graph=True)
    t3, _, _ = generate(model, prompts, 6, graph=False)
    assert torch.equal(t1, t2)
    assert torch.equal(t1, t3)  # replayed graph and eager steps agree
    # prefilling one sequence at a time runs (the MoE kernels pick plans by batch size, so
    # bits may differ from the packed prefill; the oracle test covers the values)
    t4, _, _ = generate(model, prompts, 6, graph=True, prefill_chunk=1)
    assert t4.shape == t1.shape
    assert t1.shape == (3, 6) and int(t1.min()) >= 0 and int(t1.max()) < 1000
