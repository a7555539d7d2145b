"""The Qwen3 model port, its paged KV cache and LLM.generate.

CPU: cache bookkeeping, config parsing, sampling filters.  GPU: a two-layer
model (one dense-MLP layer, one MoE layer) against a plain-torch float32
reference forward (tests/qwen3_reference.py) for the three attention paths
(initial prefill, one-token decode, prefill after a prefix), the
reference's incremental-decode comparison (tests/test_paged_attention.py:
191-213: log-softmax of the paged model vs the dense one, position by
position), batching, and LLM.generate.

Bound: log-probabilities within atol 5e-2 of the reference.  The model and
the reference round the same bf16 tensors but accumulate differently (the
exact router-size products, the GEMV, the GEMM's fp16-rounded weights), so a
bf16 activation can differ by an ulp (2^-8 relative) and that difference
travels through two layers.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

DEV = "cuda:0"
ATOL = 5e-2


def _cfg(**kw):
    from nano_vllm_metal_amd import Qwen3Config

    d = dict(hidden_size=256, num_hidden_layers=2, num_attention_heads=4,
             num_key_value_heads=2, head_dim=64, vocab_size=1024, intermediate_size=640,
             moe_intermediate_size=128, num_experts=8, num_experts_per_tok=2,
             norm_topk_prob=True, mlp_only_layers=[0], rms_norm_eps=1e-6,
             rope_theta=10000.0, max_position_embeddings=512)
    d.update(kw)
    return Qwen3Config.from_dict(d)


# ---------------------------------------------------------------- CPU


def test_config_and_sparse_layers():
    c = _cfg(num_hidden_layers=6, decoder_sparse_step=2, mlp_only_layers=[3])
    assert [i for i in range(6) if c.is_sparse(i)] == [1, 5]
    assert _cfg(head_dim=None).head_dim == 64
    assert not _cfg(num_experts=0).is_sparse(1)


def test_kv_cache_bookkeeping():
    from nano_vllm_metal_amd import PagedKVCache

    c = PagedKVCache(2, 2, 8, num_pages=6, page_size=4, dtype=torch.float32, device="cpu")
    c.add(7)
    c.add(9)
    c.reserve(7, 5)                      # 2 pages
    pages, slots = c.slot_mapping([7], 5)
    assert slots.tolist() == [0, 1, 2, 3, 0]
    assert pages.tolist() == [c.pages[7][0]] * 4 + [c.pages[7][1]]
    k = torch.arange(5 * 2 * 8, dtype=torch.float32).reshape(1, 5, 2, 8)
    c.write(1, k, -k, pages, slots)
    c.advance([7], 5)
    assert torch.equal(c.key_pages[1][c.pages[7][1], :, 0], k[0, 4])
    assert torch.equal(c.value_pages[1][c.pages[7][0], :, 3], -k[0, 3])
    c.reserve(9, 1)
    bt, lens = c.block_table([7, 9], extra=1)
    assert bt.shape == (2, 2) and bt[1, 1].item() == -1 and lens.tolist() == [6, 1]
    assert c.free_pages == 3
    c.free(7)
    assert c.free_pages == 5 and 7 not in c.pages
    with pytest.raises(RuntimeError, match="out of pages"):
        c.reserve(9, 100)


def test_sampling_filters():
    from nano_vllm_metal_amd.llm import SamplingParams, sample

    logits = torch.tensor([[0.0, 3.0, 1.0, 2.9], [5.0, 0.0, 0.0, 0.0]])
    assert sample(logits, SamplingParams()).tolist() == [1, 0]
    g = torch.Generator().manual_seed(0)
    picks = {int(sample(logits[:1], SamplingParams(temperature=1.0, top_k=2), g)[0])
             for _ in range(200)}
    assert picks == {1, 3}
    picks = {int(sample(logits[:1], SamplingParams(temperature=1.0, top_p=0.3), g)[0])
             for _ in range(100)}
    assert picks == {1}


# ---------------------------------------------------------------- GPU


def _model(seed=0, **kw):
    from nano_vllm_metal_amd import Moe, QuantizedWeights, Qwen3Model, quantize
    from nano_vllm_metal_amd.qwen3 import DenseMLP, Qwen3Layer

    c = _cfg(**kw)
    g = torch.Generator(device=DEV).manual_seed(seed)

    def qw(*shape, std=0.05):
        w = (torch.randn(shape, generator=g, device=DEV) * std).to(torch.bfloat16)
        wq, s, b = quantize(w, 64, 4)
        return QuantizedWeights(s, b, 64, 4, wq)

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g, device=DEV)).to(torch.bfloat16)

    H, D = c.hidden_size, c.head_dim
    layers = []
    for i in range(c.num_hidden_layers):
        if c.is_sparse(i):
            E, I = c.num_experts, c.moe_intermediate_size
            mlp = Moe(qw(E, H, std=0.2), qw(E, I, H), qw(E, I, H), qw(E, H, I),
                      c.num_experts_per_tok, c.norm_topk_prob)
        else:
            mlp = DenseMLP(qw(c.intermediate_size, H), qw(c.intermediate_size, H),
                           qw(H, c.intermediate_size))
        layers.append(Qwen3Layer(qw(c.num_attention_heads * D, H), qw(c.num_key_value_heads * D, H),
                                 qw(c.num_key_value_heads * D, H), qw(H, c.num_attention_heads * D),
                                 norm(D), norm(D), norm(H), norm(H), mlp))
    return Qwen3Model(c, qw(c.vocab_size, H, std=1.0), layers, norm(H), qw(c.vocab_size, H))


def _close(a, b, what):
    la = torch.log_softmax(a.float(), -1)
    lb = torch.log_softmax(b.float(), -1)
    err = (la - lb).abs().max().item()
    print(f"{what}: max |log p - log p_ref| = {err:.3g}", flush=True)
    assert err <= ATOL, f"{what}: max |log p - log p_ref| = {err:.3g}"


def _tokens(n, seed=1, vocab=1024):
    return np.random.default_rng(seed).integers(0, vocab, n).tolist()


@pytest.mark.gpu
def test_prefill_matches_reference():
    from qwen3_reference import reference_logits

    m = _model()
    toks = _tokens(12)
    cache = m.create_kv_cache(16, page_size=4)
    cache.add(0)
    got = m.forward(torch.tensor([toks], device=DEV), cache, [0], last_only=False)[0]
    _close(got, reference_logits(m, toks), "initial prefill")
    assert cache.lens[0] == 12


@pytest.mark.gpu
def test_incremental_decode_matches_reference():
    """tests/test_paged_attention.py:191-213: one token at a time through the
    paged cache (decode attention kernel) against the dense reference."""
    from qwen3_reference import reference_logits

    m = _model(1)
    toks = _tokens(10, seed=2)
    ref = reference_logits(m, toks)
    cache = m.create_kv_cache(16, page_size=4)
    cache.add(3)
    for i, t in enumerate(toks):
        got = m.forward(torch.tensor([[t]], device=DEV), cache, [3])[0]
        _close(got, ref[i], f"decode position {i}")


@pytest.mark.gpu
def test_prefill_after_prefix_matches_reference():
    """A second prompt chunk attends to the cached prefix (paged attention,
    several causal query rows)."""
    from qwen3_reference import reference_logits

    m = _model(2)
    toks = _tokens(13, seed=3)
    ref = reference_logits(m, toks)
    cache = m.create_kv_cache(16, page_size=4)
    cache.add(0)
    m.forward(torch.tensor([toks[:5]], device=DEV), cache, [0])
    got = m.forward(torch.tensor([toks[5:]], device=DEV), cache, [0], last_only=False)[0]
    _close(got, ref[5:], "chunked prefill")


@pytest.mark.gpu
def test_batched_decode_matches_single_requests():
    from qwen3_reference import reference_logits

    m = _model(3)
    prompts = [_tokens(n, seed=10 + n) for n in (3, 9, 6)]
    cache = m.create_kv_cache(32, page_size=4)
    for i, p in enumerate(prompts):
        cache.add(i)
        m.forward(torch.tensor([p[:-1]], device=DEV), cache, [i])
    last = torch.tensor([[p[-1]] for p in prompts], device=DEV)
    got = m.forward(last, cache, [0, 1, 2])
    for i, p in enumerate(prompts):
        _close(got[i], reference_logits(m, p)[-1], f"batched row {i}")


@pytest.mark.gpu
@pytest.mark.parametrize("graphs", [False, True])
def test_generate_greedy_is_the_model_argmax_chain(graphs):
    """Continuous batching (5 requests, 4 slots; two 8-token prompts prefilled
    together under a 16-token budget) with eager or graph-replayed decode
    steps gives each request the greedy chain it gets alone."""
    from nano_vllm_metal_amd import LLM, SamplingParams

    m = _model(4)
    prompts = [_tokens(n, seed=20 + i) for i, n in enumerate((5, 11, 8, 8, 8))]
    llm = LLM(m, max_num_seqs=4, max_model_len=64, page_size=4, use_graphs=graphs,
              prefill_step=16)
    outs = llm.generate(prompts, SamplingParams(max_tokens=6))
    assert [len(o.token_ids) for o in outs] == [6] * 5
    assert llm.cache.free_pages == llm.cache.num_pages
    for p, o in zip(prompts, outs):
        cache = m.create_kv_cache(16, page_size=4)
        cache.add(0)
        seq = list(p)
        logits = m.forward(torch.tensor([seq], device=DEV), cache, [0])
        chain = []
        for _ in range(6):
            t = int(torch.argmax(logits[0]))
            chain.append(t)
            logits = m.forward(torch.tensor([[t]], device=DEV), cache, [0])
        assert o.token_ids == chain
    st = llm.stats
    assert st.prefill_tokens == 40 and st.decode_tokens == 25


@pytest.mark.gpu
def test_graph_decode_matches_eager_logits():
    """Replayed decode steps give the eager step's logits (same kernels,
    same inputs) on every replay, and the capture touched no live page."""
    from nano_vllm_metal_amd import LLM

    m = _model(5)
    prompts = [_tokens(n, seed=40 + n) for n in (7, 4)]
    eager = LLM(m, max_num_seqs=2, max_model_len=32, page_size=4, use_graphs=False)
    graph = LLM(m, max_num_seqs=2, max_model_len=32, page_size=4, use_graphs=True)
    for llm in (eager, graph):
        for i, p in enumerate(prompts):
            llm.cache.add(i)
            m.forward(torch.tensor([p], device=DEV), llm.cache, [i])
    toks = [3, 17]
    for step in range(4):
        t = torch.tensor([[x] for x in toks], device=DEV)
        a = eager._decode_step(t, [0, 1]).float()
        b = graph._decode_step(t, [0, 1]).float()
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"step {step}"
        toks = [int(x) for x in torch.argmax(a, -1)]


@pytest.mark.gpu
def test_generate_sampling_stays_in_filtered_set():
    """Temperature sampling with top-k: every sampled token is among the k
    most likely of its step (checked by replaying the step), lengths hold.
    bf16 logits tie often; the filter keeps every token whose logit reaches
    the k-th largest, so a tied token counts as inside."""
    from nano_vllm_metal_amd import LLM, SamplingParams

    m = _model(6)
    prompts = [_tokens(n, seed=60 + n) for n in (6, 9)]
    llm = LLM(m, max_num_seqs=2, max_model_len=64, page_size=4, use_graphs=False)
    outs = llm.generate(prompts, SamplingParams(max_tokens=5, temperature=0.8, top_k=3))
    for p, o in zip(prompts, outs):
        assert len(o.token_ids) == 5
        cache = m.create_kv_cache(16, page_size=4)
        cache.add(0)
        logits = m.forward(torch.tensor([p], device=DEV), cache, [0])
        for t in o.token_ids:
            vals = logits[0].float()
            kth = torch.topk(vals, 3).values[-1]
            assert vals[t] >= kth, (t, float(vals[t]), torch.topk(vals, 4))
            logits = m.forward(torch.tensor([[t]], device=DEV), cache, [0])


def _row_ulp(ref):
    """bf16 ulp at each row's largest |logit| (the rounding step of the
    logits that decide the log-probabilities)."""
    top = ref.float().abs().max(-1).values.clamp_min(2.0 ** -100)
    return torch.pow(2.0, torch.floor(torch.log2(top)) - 7)


@pytest.mark.gpu
def test_generate_at_30b_a3b_dimensions():
    """Two layers at Qwen3-30B-A3B's dimensions (hidden 2048, 32 query and 4
    kv heads of 128, 128 experts, top-8 renormalised, moe_intermediate 768,
    vocabulary 151936; random int4 weights) through LLM.generate: continuous
    batching (three requests, two slots, graph-replayed decode) against the
    float32 reference forward.

    The bar is in units of the bf16 logits' own rounding step at each row's
    largest logit (about 7 here, ulp 2^-5): model and reference round the same
    bf16 tensors at the same points but sum in different orders, so logits
    may differ by a few such ulps.  Every generated token must be the
    reference's greedy choice within 4 ulps: two logits each off by up to 2
    ulps (the median bar of the prefill check below) may swap a near-tie of
    up to 4 ulps.  Prefill logits must agree within
    4 ulps per position, except where 128-way routing sits on a near-tie: the
    router logits are act-rounded values, a one-ulp difference in a layer's
    input can move a logit by one act ulp (and its probability by about two
    probability ulps), so where the k-th and (k+1)-th experts' logits lie
    within two ulps the model and the reference may pick different experts
    (ties go to the lower index in both).  Such positions are allowed only
    where the reference shows that near-tie in some layer, and at most three
    of them."""
    from nano_vllm_metal_amd import LLM, Qwen3Model, SamplingParams, qwen3_30b_a3b_config
    from qwen3_reference import reference_logits

    cfg = qwen3_30b_a3b_config(2)
    m = Qwen3Model.random(cfg, device=DEV, seed=11)
    prompts = [_tokens(n, seed=80 + n, vocab=cfg.vocab_size) for n in (24, 17, 24)]
    llm = LLM(m, max_num_seqs=2, max_model_len=64, page_size=16, prefill_step=64)
    outs = llm.generate(prompts, SamplingParams(max_tokens=6, ignore_eos=True))
    assert [len(o.token_ids) for o in outs] == [6] * 3
    assert llm.cache.free_pages == llm.cache.num_pages
    worst = 0.0
    for p, o in zip(prompts, outs):
        ref = reference_logits(m, p + o.token_ids).float()
        ulp = _row_ulp(ref)
        for i, t in enumerate(o.token_ids):
            pos = len(p) - 1 + i
            worst = max(worst, float((ref[pos].max() - ref[pos, t]) / ulp[pos]))
    print(f"30B-dims generate: worst reference logit gap of a chosen token {worst:.3g} ulps",
          flush=True)
    assert worst <= 4.0

    cache = m.create_kv_cache(8, page_size=16)
    cache.add(0)
    got = m.forward(torch.tensor([prompts[0]], device=DEV), cache, [0], last_only=False)[0]
    margins = []
    ref = reference_logits(m, prompts[0], margins).float()
    err = ((got.float() - ref).abs().max(-1).values / _row_ulp(ref)).cpu()
    near = torch.stack(margins).min(0).values
    print("30B-dims prefill: per-position max logit difference (row ulps):",
          [round(float(e), 2) for e in err], flush=True)
    print("30B-dims prefill: smallest routing logit margin per position (ulps):",
          [round(float(v), 2) for v in near], flush=True)
    bad = err > 4.0
    assert int(bad.sum()) <= 3, f"{int(bad.sum())} positions beyond 4 ulps"
    assert bool((near[bad] <= 2.0).all()), "a position beyond 4 ulps without a routing near-tie"
    assert float(err.median()) <= 2.0
