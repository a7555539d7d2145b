"""GPU parity of paged attention (nvm_paged_attention) against the oracle.

Outputs are float32 weighted averages of value rows of unit scale; the
kernels sum in float32 (as the reference does) and the oracle exactly, so the
bound is np.allclose(rtol=1e-4, atol=2e-5) on every element.  Cases follow
the reference's tests/test_paged_attention.py (dense equivalence, an empty
request, a page id of -1) and the serving shapes (Qwen3-30B-A3B: 32 query
heads, 4 kv heads, head dim 128, page 16).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention_oracle as AO

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
RTOL, ATOL = 1e-4, 2e-5
TORCH = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _run(seed, B, Hq, Hkv, D, ps, lens, L=1, dtype="bfloat16", causal=False, P=None,
         holes=0, past_pool=0, int8=False, q_scale=1.0):
    from nano_vllm_metal_amd import paged_attention

    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    mp = max(1, int(-(-lens.max() // ps)))
    P = P or B * mp + 3
    q = torch.from_numpy((rng.standard_normal((B, Hq, L, D)) * q_scale).astype(np.float32))
    kf, vf = AO.make_pool(rng, P, Hkv, ps, D)
    if int8:
        kc, ksc = AO.quantize_int8(kf)
        vc, vsc = AO.quantize_int8(vf)
        kp, vp = torch.from_numpy(kc), torch.from_numpy(vc)
        ks = torch.from_numpy(ksc[..., None])
        vs = torch.from_numpy(vsc[..., None])
    else:
        kp = torch.from_numpy(kf.astype(np.float32)).to(TORCH[dtype])
        vp = torch.from_numpy(vf.astype(np.float32)).to(TORCH[dtype])
        ks = vs = None
    bt = np.stack([rng.permutation(P)[:mp] for _ in range(B)]).astype(np.int32)
    for _ in range(holes):
        bt[rng.integers(B), rng.integers(mp)] = -1
    for _ in range(past_pool):
        bt[rng.integers(B), rng.integers(mp)] = P + int(rng.integers(1, 5))
    out = paged_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), torch.from_numpy(bt).to(DEV),
                          torch.from_numpy(lens).to(DEV), ps,
                          key_scales=None if ks is None else ks.to(DEV),
                          value_scales=None if vs is None else vs.to(DEV),
                          mask="causal" if causal else None)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.shape == (B, Hq, L, D)
    ref = AO.paged_attention(q.numpy().reshape(B * Hq, L, D), kp.float().numpy(),
                             vp.float().numpy(), bt, lens, 1.0 / np.sqrt(D), causal, Hkv, Hq,
                             None if ks is None else ks.numpy()[..., 0],
                             None if vs is None else vs.numpy()[..., 0])
    got = out.cpu().numpy().reshape(B * Hq, L, D)
    bad = ~np.isclose(got, ref, rtol=RTOL, atol=ATOL)
    assert not bad.any(), (f"{int(bad.sum())} of {bad.size} outside tolerance; "
                           f"max abs err {np.abs(got - ref).max():.3g}")
    return got, ref


# ---------------------------------------------------------------- decode kernel


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_decode_serving_shape(dtype):
    """32 requests of up to 1280 positions, 30B-A3B heads: split context."""
    rng = np.random.default_rng(11)
    lens = rng.integers(1000, 1281, 32)
    _run(100, 32, 32, 4, 128, 16, lens, dtype=dtype, holes=3)


@pytest.mark.parametrize("lens", [[1, 17, 300, 0], [64, 65, 127, 2000]])
def test_decode_ragged_contexts(lens):
    """Empty request (zeros), one position, tile and page boundaries."""
    got, _ = _run(101, 4, 32, 4, 128, 16, lens, holes=1)
    if lens[3] == 0:
        assert np.all(got[96:] == 0)


@pytest.mark.parametrize("Hq,Hkv,D", [(16, 1, 64), (48, 2, 128), (8, 8, 128), (12, 4, 64)])
def test_decode_head_groupings(Hq, Hkv, D):
    """16 query heads per kv head (one 16-row group), 24 (two groups, the
    second half full), 1 (MHA), 3."""
    _run(102, 3, Hq, Hkv, D, 16, [700, 33, 1500], dtype="float16")


@pytest.mark.parametrize("ps", [4, 128, 24])
def test_decode_page_sizes(ps):
    """Pages smaller than a 16-row subtile, larger than a tile, and not a
    power of two; page ids past the pool are skipped."""
    _run(103, 2, 32, 4, 128, ps, [500, 131], holes=2, past_pool=1)


@pytest.mark.parametrize("dtype,q_std", [("float16", 0.2), ("float16", 3.0),
                                          ("bfloat16", 3.0)])
def test_decode_query_magnitudes(dtype, q_std):
    """The float32 query enters the score MFMAs as three page-dtype parts:
    query entries of std 0.2 (the f16 third part near the subnormal range)
    and of std 3 (scores of std 3 against unit keys: a sharp softmax) both
    stay within the bound."""
    _run(111, 4, 32, 4, 128, 16, [900, 37, 1200, 5], dtype=dtype, q_scale=q_std)


def test_decode_one_request_long_context():
    _run(104, 1, 32, 4, 128, 16, [8192])


def test_decode_all_pages_missing_gives_zero():
    from nano_vllm_metal_amd import paged_attention

    q = torch.randn(2, 8, 1, 128, device=DEV)
    kp = torch.randn(4, 2, 16, 128, device=DEV).to(torch.bfloat16)
    bt = torch.full((2, 4), -1, dtype=torch.int32, device=DEV)
    lens = torch.tensor([50, 64], dtype=torch.int32, device=DEV)
    out = paged_attention(q, kp, kp.clone(), bt, lens, 16)
    assert torch.all(out == 0).item()


# ---------------------------------------------------------------- row kernel


def test_reference_unit_shape_f32():
    """tests/test_paged_attention.py:105-138 shape: D=4, page 4, float32."""
    _run(105, 1, 4, 2, 4, 4, [6], dtype="float32")
    _run(106, 3, 4, 2, 4, 4, [4, 0, 7], dtype="float32", holes=0)


@pytest.mark.parametrize("L,causal", [(3, True), (6, True), (2, False)])
def test_multi_query_rows(L, causal):
    _run(107, 2, 8, 2, 128, 16, [40, 300], L=L, causal=causal)


# ------------------------------------------------- multi-query matrix-core kernel


def test_chunk_of_256_over_1024_cached_positions():
    """Chunked prefill / prefill after a prefix at the 30B-A3B heads: four
    requests add 256 query rows each over 1024 cached positions (1280 in the
    context), causal (query row i sees j <= i + 1024), on the matrix-core
    kernel (paged_prefill.hip)."""
    _run(120, 4, 32, 4, 128, 16, [1280, 1280, 1100, 1280], L=256, causal=True, dtype="bfloat16")


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("Hq,Hkv,D,ps,L,causal", [
    (8, 8, 64, 4, 17, True),     # one query head per kv head, small pages
    (16, 8, 128, 24, 33, False),  # two per kv head, pages of 24 slots, not causal
    (16, 4, 64, 128, 70, True),  # four per kv head, pages of 128 slots
    (16, 1, 128, 16, 9, True),   # sixteen per kv head
])
def test_multi_query_matrix_core_shapes(dtype, Hq, Hkv, D, ps, L, causal):
    """Head groupings, page sizes and ragged contexts (one shorter than the
    chunk: its first rows see nothing), with missing pages and page ids past
    the pool, which the reference skips."""
    _run(121 + L, 3, Hq, Hkv, D, ps, [L + 150, L - 3, 2 * L], L=L, causal=causal, dtype=dtype,
         holes=2, past_pool=1)


def test_multi_query_query_magnitudes():
    """float32 queries far from act-representable values (three-part split)."""
    _run(130, 2, 8, 2, 128, 16, [200, 90], L=40, causal=True, dtype="bfloat16", q_scale=37.0)


def test_int8_decode():
    """paged_attention_int8_decode: codes times per-slot scales."""
    _run(108, 4, 32, 4, 128, 16, [1, 90, 600, 0], int8=True, holes=1)


def test_int8_multi_query_causal():
    _run(109, 2, 8, 4, 64, 16, [33, 100], L=4, causal=True, int8=True)


@pytest.mark.parametrize("D", [96, 256, 32])
def test_other_head_dims(D):
    _run(110, 2, 8, 2, D, 16, [77, 300])


def test_graph_replay_matches_eager():
    """The decode path (split kernel + combine) captured in a HIP graph gives
    the eager result on every replay."""
    from nano_vllm_metal_amd import paged_attention

    g = torch.Generator(device=DEV).manual_seed(5)
    B, Hq, Hkv, D, ps, mp = 8, 32, 4, 128, 16, 80
    q = torch.randn(B, Hq, 1, D, device=DEV, generator=g)
    kp = torch.randn(B * mp, Hkv, ps, D, device=DEV, generator=g).to(torch.bfloat16)
    vp = torch.randn(B * mp, Hkv, ps, D, device=DEV, generator=g).to(torch.bfloat16)
    bt = torch.randperm(B * mp, device=DEV, generator=g).to(torch.int32).reshape(B, mp)
    lens = torch.full((B,), 1200, dtype=torch.int32, device=DEV)
    eager = paged_attention(q, kp, vp, bt, lens, ps)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        paged_attention(q, kp, vp, bt, lens, ps)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = paged_attention(q, kp, vp, bt, lens, ps)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        eager2 = paged_attention(q, kp, vp, bt, lens, ps)
        torch.cuda.synchronize()
        assert torch.equal(eager2, eager)


@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float16])
def test_output_in_activation_dtype(odt):
    """out_dtype bf16/f16 is the float32 result rounded once (decode kernel
    with and without a split, and the row kernel)."""
    from nano_vllm_metal_amd import paged_attention

    g = torch.Generator(device=DEV).manual_seed(3)
    for B, L, ctx in ((32, 1, 1200), (64, 1, 2048), (2, 3, 90)):
        mp = -(-ctx // 16)
        q = torch.randn(B, 32, L, 128, device=DEV, generator=g)
        kp = torch.randn(B * mp, 4, 16, 128, device=DEV, generator=g).to(torch.bfloat16)
        vp = torch.randn(B * mp, 4, 16, 128, device=DEV, generator=g).to(torch.bfloat16)
        bt = torch.randperm(B * mp, device=DEV, generator=g).to(torch.int32).reshape(B, mp)
        lens = torch.full((B,), ctx, dtype=torch.int32, device=DEV)
        f = paged_attention(q, kp, vp, bt, lens, 16, mask="causal")
        h = paged_attention(q, kp, vp, bt, lens, 16, mask="causal", out_dtype=odt)
        assert h.dtype == odt and torch.equal(h, f.to(odt)), (B, L, ctx)


# ------------------------------------------------------------ causal prefill


def _causal_case(seed, B, L, Hq, Hkv, D, act):
    """q [B, L, Hq, D], k, v [B, L, Hkv, D] holding act-dtype values (as the
    model's q/k norm and RoPE leave them), with the f64 oracle per request."""
    rng = np.random.default_rng(seed)
    dt = torch.bfloat16 if act == "bfloat16" else torch.float16
    q = torch.from_numpy(rng.standard_normal((B, L, Hq, D)).astype(np.float32)).to(dt).float()
    k = torch.from_numpy(rng.standard_normal((B, L, Hkv, D)).astype(np.float32)).to(dt).float()
    v = torch.from_numpy(rng.standard_normal((B, L, Hkv, D)).astype(np.float32)).to(dt).float()
    return q, k, v, dt


def _causal_ref(q, k, v, b, h, scale):
    R = q.shape[2] // k.shape[2]
    return AO.dense_attention(q[b, :, h].numpy(), k[b, :, h // R].numpy(), v[b, :, h // R].numpy(),
                              scale, True)


@pytest.mark.parametrize("B,L,Hq,Hkv,D,act", [
    (2, 37, 8, 2, 64, "bfloat16"),     # ragged last query block, R=4
    (1, 130, 4, 4, 128, "float16"),    # R=1: 16 positions per wavefront
    (3, 64, 16, 1, 128, "bfloat16"),   # R=16: one position per wavefront
    (1, 1, 8, 1, 64, "bfloat16"),      # a one-token prompt
])
def test_causal_attention_matches_oracle(B, L, Hq, Hkv, D, act):
    from nano_vllm_metal_amd.attention import causal_attention

    q, k, v, dt = _causal_case(7 + L, B, L, Hq, Hkv, D, act)
    scale = D ** -0.5
    out = causal_attention(q.to(DEV), k.to(DEV), v.to(DEV), scale, dt).cpu()
    for b in range(B):
        for h in range(Hq):
            ref = _causal_ref(q, k, v, b, h, scale)
            np.testing.assert_allclose(out[b, :, h].numpy(), ref, rtol=1e-4, atol=2e-5,
                                       err_msg=f"b={b} h={h}")


def test_causal_attention_30b_heads_8x1024():
    """The 30B-A3B attention shape of the end-to-end prefill: 8 requests x
    1024 tokens, 32 query heads over 4 kv heads of dim 128; two requests
    checked against the oracle head by head, every output finite, and the
    bf16 output the float32 one rounded once."""
    from nano_vllm_metal_amd.attention import causal_attention

    B, L, Hq, Hkv, D = 8, 1024, 32, 4, 128
    q, k, v, dt = _causal_case(1234, B, L, Hq, Hkv, D, "bfloat16")
    scale = D ** -0.5
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out = causal_attention(qd, kd, vd, scale, dt)
    out_bf = causal_attention(qd, kd, vd, scale, dt, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    assert torch.equal(out.to(torch.bfloat16), out_bf)
    out = out.cpu()
    for b in (0, 7):
        for h in range(Hq):
            ref = _causal_ref(q, k, v, b, h, scale)
            np.testing.assert_allclose(out[b, :, h].numpy(), ref, rtol=1e-4, atol=2e-5,
                                       err_msg=f"b={b} h={h}")


def test_causal_attention_rejects_unsupported_shapes():
    from nano_vllm_metal_amd.attention import causal_attention

    q = torch.zeros((1, 4, 6, 96), device=DEV)
    k = torch.zeros((1, 4, 2, 96), device=DEV)
    with pytest.raises(ValueError, match="head dim"):
        causal_attention(q, k, k, 0.1, torch.bfloat16)
