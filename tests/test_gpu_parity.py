"""GPU parity of the HIP path against the CPU oracle (run on an MI355X).

Integer outputs (top-k ids, dispatch permutations) must match bit for bit;
activation-dtype outputs within the tolerances stated in helpers.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import (assert_moe_close, make_moe, qweights, to_act, to_np, to_words)
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _route_case(seed, T, H, E, k, act, gs, norm, x_std=1.0, router_std=0.02):
    rng = np.random.default_rng(seed)
    x = O.round_act(rng.standard_normal((T, H)) * x_std, act)
    wr = O.round_act(rng.standard_normal((E, H)) * router_std, act)
    router = O.quantize(wr, gs, 4, act)
    return x, router


# ---------------------------------------------------------------- router


@pytest.fixture(params=["f64", "i8"])
def route_kernel(request, monkeypatch):
    """The router's partial logits on the float64 matrix cores or, exactly,
    on the int8 ones (route_i8.hip; chosen for batches of 128 tokens or more,
    forced here for every batch)."""
    monkeypatch.setenv("NVM_ROUTE_I8", "0" if request.param == "f64" else "1")
    return request.param


@pytest.mark.parametrize("T,H,E,k,act,gs", [
    (32, 256, 16, 4, "float16", 64),       # tiny parity config
    (4, 128, 4, 2, "float16", 128),        # reference test_router_topk shape
    (1, 2048, 128, 8, "bfloat16", 64),     # 30B-A3B decode batches
    (8, 2048, 128, 8, "bfloat16", 64),
    (32, 2048, 128, 8, "bfloat16", 64),
    (64, 2048, 128, 8, "bfloat16", 64),
    (600, 2048, 128, 8, "bfloat16", 64),   # large-T router tiling
    (32, 4096, 128, 8, "bfloat16", 64),    # 235B-A22B shape
    (24, 384, 16, 4, "bfloat16", 64),      # hidden sizes that are not whole
    (24, 384, 16, 4, "float16", 128),      # 128-column blocks: one hidden split
    (24, 640, 16, 4, "float16", 64),
    (300, 1152, 64, 6, "bfloat16", 128),   # nine 128-column blocks
    (200, 512, 40, 4, "bfloat16", 64),     # experts not a multiple of 16
    (130, 1024, 512, 8, "float16", 64),    # four 128-expert ranges
])
@pytest.mark.parametrize("norm", [False, True])
def test_route_bit_exact(T, H, E, k, act, gs, norm, route_kernel):
    from nano_vllm_metal_amd import route_topk

    x, router = _route_case(1000 + T + H + E, T, H, E, k, act, gs, norm)
    _, probs_ref, ids_ref, sc_ref = O.route_topk(x, *router, gs, k, norm, act)
    w = qweights(router, act, gs, DEV)
    probs, ids, scores = route_topk(to_act(x, act, DEV), w, k, norm)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ids_ref), "top-k ids differ"
    assert np.array_equal(to_np(probs), probs_ref), "probs differ"
    assert np.array_equal(to_np(scores), sc_ref), "scores differ"


@pytest.mark.parametrize("act", ["bfloat16", "float16"])
def test_route_wide_exponent_range(act, route_kernel):
    """Activations over many binades -- zero rows, values 2^-30 and 2^-60 (bf16)
    below their neighbours, subnormals, large values -- take several exponent
    bands in the int8 router; ids, probabilities and scores must still equal
    the oracle's exactly rounded ones, as the float64 kernel's do."""
    from nano_vllm_metal_amd import route_topk

    T, H, E, k, gs = 40, 1024, 128, 8, 64
    bf = act == "bfloat16"
    rng = np.random.default_rng(77)
    x = rng.standard_normal((T, H))
    x[1] = 0.0                                   # no band at all
    x[2, ::7] *= 2.0 ** (-30 if bf else -12)     # two bands
    x[3, ::5] *= 2.0 ** (-60 if bf else -20)     # subnormal fp16 / far below (bf16)
    x[3, 1::5] *= 2.0 ** (-30 if bf else -10)    # three bands
    x[4, ::3] = 0.0
    x[5, 10] = 2.0 ** (-130 if bf else -23)      # one subnormal
    x[6] *= 2.0 ** (-100 if bf else -8)          # a whole row far from 1
    x[7, ::11] *= 2.0 ** 12                      # large values
    x[17:33] *= 2.0 ** -20 if bf else 1.0        # a tile of small rows next to normal ones
    x = O.round_act(x, act)
    wr = O.round_act(rng.standard_normal((E, H)) * 0.02, act)
    router = O.quantize(wr, gs, 4, act)
    _, probs_ref, ids_ref, sc_ref = O.route_topk(x, *router, gs, k, True, act)
    probs, ids, scores = route_topk(to_act(x, act, DEV), qweights(router, act, gs, DEV), k, True)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ids_ref), "top-k ids differ"
    assert np.array_equal(to_np(probs), probs_ref), "probs differ"
    assert np.array_equal(to_np(scores), sc_ref), "scores differ"


@pytest.mark.parametrize("T,E,k", [(1, 128, 8), (5, 128, 8), (32, 128, 8), (64, 128, 8),
                                   (65, 128, 8), (700, 128, 8), (130, 64, 6), (131, 40, 4),
                                   (300, 512, 8)])
def test_route_and_dispatch_matches_oracle(T, E, k, route_kernel):
    """One call: routing plus the stable sort (single launch for T <= 64; for
    the int8 router with E <= 128, routing in one launch per 16 tokens and the
    sort from its per-block histograms -- ragged last blocks, one 64-expert
    range, expert counts not a multiple of 16)."""
    from nano_vllm_metal_amd import route_and_dispatch

    H, act, gs = 2048, "bfloat16", 64
    x, router = _route_case(3000 + T + E, T, H, E, k, act, gs, True)
    _, _, ids_ref, sc_ref = O.route_topk(x, *router, gs, k, True, act)
    off_ref, srt_ref = O.dispatch(ids_ref, E)
    ids, scores, off, srt = route_and_dispatch(to_act(x, act, DEV), qweights(router, act, gs, DEV),
                                               k, True)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    assert np.array_equal(to_np(scores), sc_ref)
    assert np.array_equal(off.cpu().numpy(), off_ref)
    assert np.array_equal(srt.cpu().numpy(), srt_ref)


def test_route_ties_pick_lower_index():
    """All-zero router weights: every prob is 1/E, ids must be 0..k-1."""
    from nano_vllm_metal_amd import QuantizedWeights, route_topk

    T, H, E, k = 5, 256, 16, 4
    x = torch.randn(T, H, device=DEV).to(torch.bfloat16)
    w = QuantizedWeights(torch.zeros(E, H // 64, dtype=torch.bfloat16, device=DEV),
                         torch.zeros(E, H // 64, dtype=torch.bfloat16, device=DEV), 64, 4,
                         torch.zeros(E, H // 8, dtype=torch.int32, device=DEV))
    probs, ids, scores = route_topk(x, w, k, norm_topk_prob=True)
    assert ids.tolist() == [list(range(k))] * T
    assert torch.all(probs == probs[0, 0]).item()
    assert torch.all(scores.float() == 0.25).item()


def test_quantized_matmul_identity_known_answer():
    """Identity activations return the dequantised rows (test_quantized_matmul.py:13-14)."""
    from nano_vllm_metal_amd import quantized_matmul

    for act, gs in (("float16", 128), ("bfloat16", 128), ("bfloat16", 64)):
        rng = np.random.default_rng(7)
        w = O.round_act(rng.standard_normal((5, gs)), act)
        wq, s, b = O.quantize(w, gs, 4, act)
        eye = np.eye(gs)
        out = quantized_matmul(to_act(s, act, DEV), to_act(b, act, DEV), gs, 4,
                               to_act(eye, act, DEV), to_words(wq, DEV), transpose_b=True)
        ref = O.round_act(O.dequantize(wq, s, b, gs).T, act)
        assert np.array_equal(to_np(out), ref)


# Router-sized products (up to 512 outputs over up to 64 rows, or output
# widths the products do not tile): float64 sums, one rounding -> bit-exact.
# N a multiple of 512 splits the sums over a block's four wavefronts.
@pytest.mark.parametrize("M,N,K,act,gs", [(3, 128, 5, "float16", 128), (300, 512, 100, "bfloat16", 64),
                                          (7, 2048, 128, "bfloat16", 64),
                                          (37, 1024, 200, "float16", 128),
                                          (1, 4096, 512, "bfloat16", 64),
                                          (20, 640, 48, "bfloat16", 64)])
def test_quantized_matmul_matches_oracle(M, N, K, act, gs):
    from nano_vllm_metal_amd import quantized_matmul

    rng = np.random.default_rng(M * N + K)
    a = O.round_act(rng.standard_normal((M, N)), act)
    w = O.round_act(rng.standard_normal((K, N)), act)
    wq, s, b = O.quantize(w, gs, 4, act)
    out = quantized_matmul(to_act(s, act, DEV), to_act(b, act, DEV), gs, 4, to_act(a, act, DEV),
                           to_words(wq, DEV), transpose_b=True)
    assert np.array_equal(to_np(out), O.quantized_matmul(a, wq, s, b, gs, act))


# Dense projections (more than 512 outputs, or more than 64 rows) run on the
# expert GEMV (N <= 4096; up to 32 rows, or up to 512 while the GEMM grid
# would be smaller than the chip) or the GEMM, accumulating in float32 like
# quantized_matmul.metal:25-44.  The
# GEMV's sums equal the unrounded dequantised products; the GEMM rounds each
# dequantised weight to fp16 (single rounding of q*s + b) before its fp16
# MFMA, 2^-12 relative, below the output rounding of either activation dtype.
# Both are held to the tolerance against the exactly rounded oracle (outputs
# are of unit scale, so the mean error is taken relative to the largest
# output), and most elements must equal the exactly rounded result of their
# own numerics.
@pytest.mark.parametrize("M,N,K,act,gs,path", [
    (1, 2048, 4096, "bfloat16", 64, "gemv"),     # four-group slices, aligned scales
    (7, 2048, 1024, "float16", 128, "gemv"),     # group 128
    (16, 4096, 2048, "bfloat16", 128, "gemv"),   # eight-group slices, full chunk
    (3, 1024, 528, "bfloat16", 64, "gemv"),      # output tile past the last row
    (17, 2048, 768, "bfloat16", 64, "gemv"),     # two chunks, the second of one row
    (300, 1024, 4096, "float16", 64, "gemv"),    # 19 chunks (GEMM grid of 48 blocks)
    (5, 6144, 1024, "bfloat16", 128, "gemm"),    # N the GEMV does not slice
    (600, 1024, 1024, "float16", 64, "gemm"),    # beyond 512 rows, ragged last tile
    (700, 2048, 768, "bfloat16", 64, "gemm"),
    (65, 2048, 512, "bfloat16", 64, "gemv"),     # narrow output beyond 64 rows
    (300, 512, 96, "bfloat16", 64, "gemv"),
    (4096, 2048, 128, "float16", 128, "gemm"),
    (600, 768, 1024, "bfloat16", 128, "gemm"),   # 6 groups a row: windows of 2-byte loads
    (520, 192, 1024, "float16", 64, "gemm"),     # 3 k-steps: the last one after the pairs
    (600, 1024, 528, "bfloat16", 64, "gemm"),    # last n-tile of 16 columns (epilogue bound)
])
def test_quantized_matmul_dense_products(M, N, K, act, gs, path):
    from nano_vllm_metal_amd import quantized_matmul

    rng = np.random.default_rng(M * 7 + N + K)
    a = O.round_act(rng.standard_normal((M, N)), act)
    w = O.round_act(rng.standard_normal((K, N)) * 0.02, act)
    wq, s, b = O.quantize(w, gs, 4, act)
    out = quantized_matmul(to_act(s, act, DEV), to_act(b, act, DEV), gs, 4, to_act(a, act, DEV),
                           to_words(wq, DEV), transpose_b=True)
    ref = O.quantized_matmul(a, wq, s, b, gs, act)
    assert_moe_close(out, ref, act, f"quantized_matmul {M}x{N}x{K}", mae_rel=True)
    if path == "gemm":
        wd = O.round_act(O.dequantize(wq, s, b, gs), "float16")
        ref = O.round_act(np.asarray(a, np.float64) @ wd.T, act)
    same = np.mean(to_np(out) == ref)
    assert same > 0.9, f"{path}: {same:.3f} of the outputs equal the rounded exact result"


@pytest.mark.parametrize("act", ["float16", "bfloat16"])
@pytest.mark.parametrize("gs", [64, 128])
def test_torch_quantizer_on_gpu(act, gs):
    """The MLX affine quantizer that builds every benchmark and test weight set,
    run on the GPU, against the same code on the CPU and the oracle's
    quantizer.  Float32 division on the GPU is not always correctly rounded,
    so a code whose (w - b) / s lies within an ulp of a half-integer may round
    the other way: such codes are allowed, one step apart and only at such
    near-ties; scales and biases must agree in nearly every group."""
    from nano_vllm_metal_amd import quantize

    rng = np.random.default_rng(33 + gs)
    w = O.round_act(rng.standard_normal((96, 8 * gs)) * 0.02, act)
    dt = torch.float16 if act == "float16" else torch.bfloat16
    wt = torch.from_numpy(w.astype(np.float32)).to(dt)
    g_wq, g_s, g_b = (t.cpu() for t in quantize(wt.to(DEV), gs, 4))
    c_wq, c_s, c_b = quantize(wt, gs, 4)
    sb_same = (g_s.view(torch.int16) == c_s.view(torch.int16)) & \
              (g_b.view(torch.int16) == c_b.view(torch.int16))
    assert float(sb_same.float().mean()) > 0.99
    g_codes = O.unpack_nibbles(g_wq.numpy().view(np.uint32))
    c_codes = O.unpack_nibbles(c_wq.numpy().view(np.uint32))
    diff = (g_codes != c_codes) & np.repeat(sb_same.numpy(), gs, axis=1)
    assert diff.mean() < 1e-3
    if diff.any():
        s64 = np.repeat(c_s.float().numpy().astype(np.float64), gs, axis=1)
        b64 = np.repeat(c_b.float().numpy().astype(np.float64), gs, axis=1)
        x = ((w - b64) / s64)[diff]
        assert np.all(np.abs(x - np.floor(x) - 0.5) < 1e-4)
        assert np.all(np.abs(g_codes[diff].astype(np.int64) - c_codes[diff].astype(np.int64)) == 1)
    # against the oracle's quantizer, as the CPU test checks the CPU path
    owq, os_, ob = O.quantize(w, gs, 4, act)
    s_t = g_s.float().numpy().astype(np.float64)
    b_t = g_b.float().numpy().astype(np.float64)
    assert np.mean(s_t == os_) > 0.95 and np.mean(b_t == ob) > 0.95
    same = np.repeat((s_t == os_) & (b_t == ob), gs, axis=1)
    assert np.mean(g_codes[same] == O.unpack_nibbles(owq)[same]) > 0.999


# ---------------------------------------------------------------- dispatch


@pytest.mark.parametrize("n,E", [(0, 8), (1, 1), (256, 128), (100, 3), (32768, 128), (5000, 512),
                                 (4096, 1)])
def test_dispatch_matches_stable_argsort(n, E):
    from nano_vllm_metal_amd import moe_dispatch

    rng = np.random.default_rng(n + E)
    ids = rng.integers(0, E, size=n).astype(np.int32)
    off, srt = moe_dispatch(torch.from_numpy(ids).to(DEV), E)
    off_ref, srt_ref = O.dispatch(ids, E)
    assert np.array_equal(off.cpu().numpy(), off_ref)
    assert np.array_equal(srt.cpu().numpy(), srt_ref)


def test_dispatch_skewed_and_out_of_range():
    from nano_vllm_metal_amd import moe_dispatch

    E = 128
    rng = np.random.default_rng(5)
    ids = np.where(rng.random(20000) < 0.9, 3, rng.integers(0, E, 20000)).astype(np.int32)
    off, srt = moe_dispatch(torch.from_numpy(ids).to(DEV), E)
    off_ref, srt_ref = O.dispatch(ids, E)
    assert np.array_equal(off.cpu().numpy(), off_ref)
    assert np.array_equal(srt.cpu().numpy(), srt_ref)
    # ids outside [0, E) are dropped; the rest keep their stable order
    bad = ids.copy()
    bad[::7] = E + 5
    bad[1::11] = -1
    off, srt = moe_dispatch(torch.from_numpy(bad).to(DEV), E)
    keep = np.nonzero((bad >= 0) & (bad < E))[0]
    o2, s2 = O.dispatch(bad[keep], E)
    assert np.array_equal(off.cpu().numpy(), o2)
    assert np.array_equal(srt.cpu().numpy()[: len(keep)], keep[s2])


# ---------------------------------------------------------------- grouped linear


@pytest.mark.parametrize("regime", ["decode", "prefill"])
def test_grouped_expert_linear_reference_shape(regime):
    """test_moe.py:19-49 shape: x [2,3,128], 3 experts of [64,128], group 128."""
    from nano_vllm_metal_amd import grouped_expert_linear

    act, gs = "float16", 128
    rng = np.random.default_rng(1)
    x = O.round_act(rng.standard_normal((2, 3, 128)) * 0.25, act)
    w = O.round_act(rng.standard_normal((3, 64, 128)) * 0.25, act)
    wq, s, b = O.quantize(w, gs, 4, act)
    ids = np.array([[2, 0, 1], [1, 2, 0]], dtype=np.int32)
    out = grouped_expert_linear(to_act(x, act, DEV), qweights((wq, s, b), act, gs, DEV),
                                torch.from_numpy(ids).to(DEV), regime=regime)
    ref = O.grouped_expert_linear(x, wq, s, b, gs, ids, act)
    assert out.shape == (2, 3, 64)
    assert_moe_close(out, ref, act, f"grouped linear {regime}")


@pytest.mark.parametrize("regime", ["decode", "prefill"])
@pytest.mark.parametrize("n,D,O_,E,act", [(200, 512, 256, 8, "bfloat16"), (77, 768, 2048, 16, "bfloat16"),
                                          (300, 256, 128, 4, "float16")])
def test_grouped_expert_linear_matches_oracle(regime, n, D, O_, E, act):
    from nano_vllm_metal_amd import grouped_expert_linear

    gs = 64
    rng = np.random.default_rng(n + D)
    x = O.round_act(rng.standard_normal((n, D)), act)
    w = O.round_act(rng.standard_normal((E, O_, D)) * 0.02, act)
    wq, s, b = O.quantize(w, gs, 4, act)
    ids = rng.integers(0, E, n).astype(np.int32)
    out = grouped_expert_linear(to_act(x, act, DEV), qweights((wq, s, b), act, gs, DEV),
                                torch.from_numpy(ids).to(DEV), regime=regime)
    ref = O.grouped_expert_linear(x, wq, s, b, gs, ids, act)
    assert_moe_close(out, ref, act, f"grouped linear {regime}")


# ---------------------------------------------------------------- full block


def _moe_case(seed, T, H, E, I, act, gs=64):
    if E * I * H > (1 << 24):
        # 30B/235B expert shapes: weights drawn in the packed domain (seconds
        # instead of minutes of float quantisation)
        return O.make_packed_inputs(seed, T, H, E, I, act, gs)
    return O.make_inputs(seed, T, H, E, I, act, gs)


def _check_moe(x, weights, k, norm, act, gs, regime="auto", rows=None):
    moe = make_moe(weights, act, gs, k, norm, DEV)
    moe.regime = regime
    y, ids, scores = moe.forward(to_act(x, act, DEV), return_routing=True)
    torch.cuda.synchronize()
    sel = slice(None) if rows is None else rows
    y_ref, ids_ref, sc_ref = O.moe_forward(x[sel], weights, k, norm, act, gs)
    assert np.array_equal(ids.cpu().numpy()[sel], ids_ref), "ids differ"
    assert np.array_equal(to_np(scores)[sel], sc_ref), "scores differ"
    return assert_moe_close(to_np(y)[sel], y_ref, act, f"moe {regime}")


@pytest.mark.parametrize("regime", ["auto", "decode", "prefill"])
def test_moe_tiny_config(regime):
    x, w = _moe_case(11, 32, 256, 16, 128, "float16")
    _check_moe(x, w, 4, True, "float16", 64, regime)


@pytest.mark.parametrize("regime", ["decode", "prefill"])
def test_moe_reference_test_shape(regime):
    """test_moe.py:93-131 shape: hidden 128, inter 128, 3 experts, top-2, renorm, g128."""
    act, gs = "float16", 128
    rng = np.random.default_rng(3)
    s = 0.25
    x = O.round_act(rng.standard_normal((6, 128)) * s, act)
    w = {"router": O.quantize(O.round_act(rng.standard_normal((3, 128)) * s, act), gs, 4, act),
         "gate": O.quantize(O.round_act(rng.standard_normal((3, 128, 128)) * s, act), gs, 4, act),
         "up": O.quantize(O.round_act(rng.standard_normal((3, 128, 128)) * s, act), gs, 4, act),
         "down": O.quantize(O.round_act(rng.standard_normal((3, 128, 128)) * s, act), gs, 4, act)}
    _check_moe(x, w, 2, True, act, gs, regime)


@pytest.mark.parametrize("T", [1, 8, 32, 64])
def test_moe_30b_decode(T):
    x, w = _moe_case(100 + T, T, 2048, 128, 768, "bfloat16")
    _check_moe(x, w, 8, True, "bfloat16", 64, "auto")


@pytest.mark.parametrize("T,E", [(1, 128), (8, 128), (32, 128), (64, 128), (16, 64), (40, 512),
                                 (3, 1)])
@pytest.mark.parametrize("static", ["0", "1"])
def test_moe_decode_expert_major_and_dealt(T, E, static, monkeypatch):
    """The decode products (K 2048 and 768) as expert-major blocks (weights
    requested before the routing; blocks of untouched experts end at once)
    and as dealt units, each forced at every batch size: few touched experts,
    four blocks per expert (E = 64), more blocks than CUs (E = 512), one
    expert over 48 blocks."""
    monkeypatch.setenv("NVM_GEMV_STATIC", static)
    x, w = _moe_case(150 + T + E, T, 2048, E, 768, "bfloat16")
    _check_moe(x, w, min(8, E), True, "bfloat16", 64, "decode")


@pytest.mark.parametrize("H,I,T_full", [(2048, 768, 64), (4096, 1536, 32)])
def test_moe_decode_is_batch_invariant(H, I, T_full):
    """A token's output does not depend on the batch around it: the decode
    products deal their units (and halves of units) to wavefronts by the
    batch's routing, but sum every output in one fixed order."""
    w = _packed_weights(110 if H == 2048 else 300, H, 128, I, "bfloat16")
    x = O.round_act(np.random.default_rng(111).standard_normal((T_full, H)), "bfloat16")
    moe = make_moe(w, "bfloat16", 64, 8, True, DEV)
    moe.regime = "decode"
    xs = to_act(x, "bfloat16", DEV)
    full = moe.forward(xs)
    for T in (1, 5, T_full // 2):
        part = moe.forward(xs[:T].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(part, full[:T]), f"T={T} differs from the first rows of T={T_full}"


@pytest.mark.parametrize("T", [1, 5, 8, 12])
@pytest.mark.parametrize("act", ["bfloat16", "float16"])
def test_moe_decode_routing_ties(T, act):
    """The routing that the decode products finalise (one token a wavefront
    up to eight tokens, four a wavefront above): an all-zero router gives
    every expert probability 1/E, so top-k is experts 0..k-1 and each score
    1/k; router rows equal in threes tie each token's experts in groups of
    three at distinct levels, where the lower index must win inside a group."""
    E, H, I, k, gs = 128, 256, 128, 8, 64
    x, w = _moe_case(170 + T, T, H, E, I, act)
    wq, s, b = w["router"]
    w0 = dict(w, router=(np.zeros_like(wq), np.zeros_like(s), np.zeros_like(b)))
    moe = make_moe(w0, act, gs, k, True, DEV)
    moe.regime = "decode"
    _, ids, scores = moe.forward(to_act(x, act, DEV), return_routing=True)
    torch.cuda.synchronize()
    assert ids.cpu().tolist() == [list(range(k))] * T
    assert torch.all(scores.float() == 1.0 / k).item()
    _check_moe(x, w0, k, True, act, gs, "decode")
    # levels 2^-6 .. apart so their probabilities stay distinct after rounding
    lv = O.round_act(np.random.default_rng(171).permutation(np.arange(E // 3 + 1)) * 2.0 ** -6, act)
    rb = np.repeat(lv[np.arange(E) // 3][:, None], b.shape[1], axis=1)
    w3 = dict(w, router=(np.zeros_like(wq), np.zeros_like(s), rb.astype(b.dtype)))
    _check_moe(x, w3, k, True, act, gs, "decode")
    moe3 = make_moe(w3, act, gs, k, True, DEV)
    moe3.regime = "decode"
    _, ids3, _ = moe3.forward(to_act(x, act, DEV), return_routing=True)
    ids3 = ids3.cpu().numpy()
    for t in range(T):
        g = ids3[t] // 3
        for j in range(k - 1):
            if g[j] == g[j + 1]:
                assert ids3[t, j] < ids3[t, j + 1], f"token {t}: tie inside group {g[j]} misordered"


@pytest.mark.parametrize("T,H,I,act", [(1, 2048, 768, "bfloat16"), (3, 2048, 768, "bfloat16"),
                                       (8, 2048, 768, "float16"), (16, 2048, 768, "bfloat16"),
                                       (32, 2048, 768, "bfloat16"), (1, 4096, 1536, "bfloat16"),
                                       (8, 4096, 1536, "bfloat16")])
def test_moe_decode_down_combine_is_bit_identical(T, H, I, act, monkeypatch):
    """The down product with the combine in its epilogue (one block per 16
    columns of y over every pair) against the down product followed by the
    combine launch: the same y bits, routing and scores, forced both ways
    (NVM_DOWN_COMBINE) at batch sizes up to its 256-pair limit, both dtypes
    and the 235B shape; the fused output also checked against the oracle."""
    x, w = _moe_case(900 + T + H, T, H, 128, I, act)
    moe = make_moe(w, act, 64, 8, True, DEV)
    moe.regime = "decode"
    xs = to_act(x, act, DEV)
    outs = []
    for fused in ("0", "1"):
        monkeypatch.setenv("NVM_DOWN_COMBINE", fused)
        y, ids, sc = moe.forward(xs, return_routing=True)
        torch.cuda.synchronize()
        outs.append((y.clone(), ids.clone(), sc.clone()))
    print(f"down+combine T={T} H={H} {act}", flush=True)
    for a, b, what in zip(outs[0], outs[1], ("y", "ids", "scores")):
        assert torch.equal(a, b), f"{what}: fused down+combine differs from down then combine"
    y_ref, _, _ = O.moe_forward(x, w, 8, True, act, 64)
    assert_moe_close(to_np(outs[1][0]), y_ref, act, "moe down+combine")


@pytest.mark.parametrize("T,E,act,force", [(32, 128, "bfloat16", ""), (64, 128, "bfloat16", ""),
                                           (16, 128, "bfloat16", ""),
                                           (40, 128, "float16", ""), (8, 128, "bfloat16", "1"),
                                           (1, 128, "bfloat16", "1"), (32, 64, "bfloat16", "1")])
def test_moe_decode_fused_down_is_bit_identical(T, E, act, force, monkeypatch):
    """The decode gate/up and down products in one launch (two expert-major
    blocks per expert, each over one half of the down reduction, h kept in
    LDS; the combine adds the halves) against the two launches: the same y
    bits, routing and scores, forced both ways (NVM_FUSED_DOWN) where it is
    chosen and below its batch threshold (few rows, many untouched experts,
    E = 64); the combine with the residual add and RMSNorm after the block
    likewise; the fused output also checked against the oracle."""
    from nano_vllm_metal_amd.fused import moe_residual_rms_norm

    x, w = _moe_case(950 + T + E, T, 2048, E, 768, act)
    moe = make_moe(w, act, 64, 8, True, DEV)
    moe.regime = "decode"
    xs = to_act(x, act, DEV)
    g = torch.Generator(device=DEV).manual_seed(T)
    h = (torch.randn(T, 2048, device=DEV, generator=g) * 2).to(xs.dtype)
    nw = (1 + 0.1 * torch.randn(2048, device=DEV, generator=g)).to(xs.dtype)
    outs = []
    for fused in ("0", force or "1"):
        if force or fused == "0":
            monkeypatch.setenv("NVM_FUSED_DOWN", fused)
        else:
            monkeypatch.delenv("NVM_FUSED_DOWN", raising=False)
        y, ids, sc = moe.forward(xs, return_routing=True)
        h2, x2 = moe_residual_rms_norm(moe, xs, h, nw, 1e-6)
        torch.cuda.synchronize()
        outs.append((y.clone(), ids.clone(), sc.clone(), h2.clone(), x2.clone()))
    print(f"fused down T={T} E={E} {act} force={force!r}", flush=True)
    for a, b, what in zip(outs[0], outs[1], ("y", "ids", "scores", "h_out", "x_out")):
        assert torch.equal(a, b), f"{what}: fused gate/up + down differs from two launches"
    y_ref, _, _ = O.moe_forward(x, w, min(8, E), True, act, 64)
    assert_moe_close(to_np(outs[1][0]), y_ref, act, "moe fused down")


@pytest.mark.parametrize("T", [20, 40, 64])
def test_moe_decode_fused_down_skewed(T, monkeypatch):
    """Zipf(1.1) routing through the fused decode products: popular experts
    take 17-20 rows (two chunks staged in one phase) or more (several
    phases), beside experts of one chunk, whose two wavefronts per SIMD
    share a tile's halves.  The same y bits, routing and scores as the two
    launches, and y against the oracle."""
    H, E, I, act = 2048, 128, 768, "bfloat16"
    x, w = _skewed_case(960 + T, T, H, E, I, act)
    _, _, ids_ref, _ = O.route_topk(x, *w["router"], 64, 8, True, act)
    counts = np.bincount(ids_ref.reshape(-1), minlength=E)
    assert counts.max() > 16 and (counts[counts > 0] <= 16).any(), counts
    moe = make_moe(w, act, 64, 8, True, DEV)
    moe.regime = "decode"
    xs = to_act(x, act, DEV)
    outs = []
    for fused in ("0", "1"):
        monkeypatch.setenv("NVM_FUSED_DOWN", fused)
        y, ids, sc = moe.forward(xs, return_routing=True)
        torch.cuda.synchronize()
        outs.append((y.clone(), ids.clone(), sc.clone()))
    print(f"fused down skewed T={T}: rows per expert max {counts.max()}, "
          f"{int(((counts > 16) & (counts <= 20)).sum())} of 17-20, "
          f"{int((counts > 20).sum())} above 20", flush=True)
    for a, b, what in zip(outs[0], outs[1], ("y", "ids", "scores")):
        assert torch.equal(a, b), f"{what}: fused gate/up + down differs from two launches"
    y_ref, _, _ = O.moe_forward(x, w, 8, True, act, 64)
    assert_moe_close(to_np(outs[1][0]), y_ref, act, "moe fused down skewed")


def test_moe_235b_decode():
    """H4096 I1536: gate/up through the eight-group slice GEMV (KS 8), down
    through six-group slices in four k-slices."""
    w = _packed_weights(300, 4096, 128, 1536, "bfloat16")
    x = O.round_act(np.random.default_rng(303).standard_normal((32, 4096)), "bfloat16")
    _check_moe(x, w, 8, True, "bfloat16", 64, "decode")


def test_moe_30b_decode_group128():
    """Group size 128: the decode GEMV's general scale windows (two groups per
    128-code pair)."""
    x, w = _moe_case(400, 32, 2048, 128, 768, "bfloat16", gs=128)
    _check_moe(x, w, 8, False, "bfloat16", 128, "decode")


@pytest.mark.parametrize("H,I,act,gs", [(384, 256, "bfloat16", 64), (384, 256, "float16", 128),
                                         (640, 320, "float16", 64)])
def test_moe_odd_slice_widths(H, I, act, gs):
    """H384: six-group gate/up slices in one k-slice; with group 128 every
    other row's scale window starts mid-dword (three values per row).  H640:
    two-group slices in five k-slices (five wavefronts per block), and the
    down product (five groups per row, no GEMV slicing) on the GEMM."""
    x, w = _moe_case(500 + H + gs, 24, H, 16, I, act, gs=gs)
    _check_moe(x, w, 4, True, act, gs, "decode")


def _skewed_case(seed, T, H, E, I, act, s=1.1, gs=64):
    """Zipf(s) expert popularity: one 64-wide activation group held at 1.0 and
    log-popularity offsets in those router columns."""
    x, w = O.make_inputs(seed, T, H, E, I, act, gs)
    x = np.array(x)
    x[:, :64] = 1.0
    rng = np.random.default_rng(seed + 1)
    wr = O.round_act(rng.standard_normal((E, H)) * 0.02, act)
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    wr[:, :64] = O.round_act(np.log(p / p.sum())[:, None] / 64.0, act)
    w["router"] = O.quantize(wr, gs, 4, act)
    return x, w


@pytest.mark.parametrize("T,E,k,regime", [(16, 512, 8, "decode"), (20, 1, 1, "decode"),
                                          (20, 1, 1, "prefill"), (40, 64, 6, "auto")])
def test_moe_expert_count_extremes(T, E, k, regime):
    """The most experts the kernels take (512), a single expert, and a top-k
    that is not a power of two."""
    x, w = _moe_case(600 + E + k, T, 256, E, 128, "bfloat16")
    _check_moe(x, w, k, True, "bfloat16", 64, regime)


@pytest.mark.parametrize("T,regime", [(300, "decode"), (5, "prefill")])
def test_moe_forced_regimes(T, regime):
    """The decode GEMV on a prefill-sized batch (many chunks per expert and
    units per block), the prefill GEMM on a handful of tokens."""
    x, w = _moe_case(700 + T, T, 256, 16, 128, "bfloat16")
    _check_moe(x, w, 4, False, "bfloat16", 64, regime)


@pytest.mark.parametrize("regime", ["decode", "prefill"])
def test_moe_skewed_routing(regime):
    """Zipf(1.1) popularity: the favourite expert takes many 128-row tiles,
    rare experts one row or none."""
    x, w = _skewed_case(800, 512, 256, 16, 128, "bfloat16")
    _, _, ids, _ = O.route_topk(x, *w["router"], 64, 4, True, "bfloat16")
    counts = np.bincount(ids.reshape(-1), minlength=16)
    assert counts.max() >= 3 * counts.mean(), counts  # the case is skewed
    _check_moe(x, w, 4, True, "bfloat16", 64, regime)


def test_moe_30b_prefill_512_all_rows():
    """T=512 at the 30B shape through the prefill GEMM, every row checked."""
    x, w = _moe_case(200, 512, 2048, 128, 768, "bfloat16")
    _check_moe(x, w, 8, True, "bfloat16", 64, "prefill")


# Large prefill batches (test_moe.py:93-131 pattern: ids compared exactly,
# outputs within tolerance).  Routing and the dispatch permutation are checked
# for every token; the block output on sampled rows: every row of the first
# and last 128-row tile of the most popular expert (its first and last GEMM
# m-tiles) and a random sample of the rest.
_WEIGHTS = {}


def _packed_weights(seed, H, E, I, act, gs=64):
    key = (seed, H, E, I, act, gs)
    if key not in _WEIGHTS:
        # (30B: 0.3 GB packed, 235B: 1.2 GB; the tests of a shape share them)
        _WEIGHTS[key] = O.make_packed_inputs(seed, 1, H, E, I, act, gs)[1]
    return _WEIGHTS[key]


def _zipf_router(seed, H, E, act, s=1.1, gs=64):
    """Zipf(s) expert popularity: with one 64-wide activation group held at 1.0,
    the first group of router row e holds log(p_e) / 64 (p_e ~ e^-s), so that
    group adds log-popularity offsets to the logits.  A token picks an expert
    at most once, so the most popular experts saturate near one pick per token
    (the capped Zipf of the 30B-A3B prefill workload)."""
    rng = np.random.default_rng(seed)
    wr = O.round_act(rng.standard_normal((E, H)) * 0.02, act)
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    wr[:, :64] = O.round_act(np.log(p / p.sum())[:, None] / 64.0, act)
    return O.quantize(wr, gs, 4, act)


def _prefill_rows(ids, E, T, seed, n_random=48, tile=128):
    counts = np.bincount(ids.reshape(-1), minlength=E)
    hot = int(np.argmax(counts))
    toks = np.nonzero((ids == hot).any(axis=1))[0]  # ascending: its slot order
    last = len(toks) - ((len(toks) - 1) % tile + 1)
    rng = np.random.default_rng(seed)
    rows = np.concatenate([toks[:tile], toks[last:], rng.integers(0, T, n_random)])
    return np.unique(rows), counts


def _check_prefill(x, w, k, act, gs, seed):
    from nano_vllm_metal_amd import route_and_dispatch

    T = x.shape[0]
    E = w["router"][0].shape[0]
    _, _, ids_ref, sc_ref = O.route_topk(x, *w["router"], gs, k, True, act)
    off_ref, srt_ref = O.dispatch(ids_ref, E)
    xt = to_act(x, act, DEV)
    moe = make_moe(w, act, gs, k, True, DEV)
    y, ids, scores = moe.forward(xt, return_routing=True)
    ids2, _, off, srt = route_and_dispatch(xt, moe.w_router, k, True)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), ids_ref), "ids differ"
    assert np.array_equal(to_np(scores), sc_ref), "scores differ"
    assert np.array_equal(ids2.cpu().numpy(), ids_ref), "route_and_dispatch ids differ"
    assert np.array_equal(off.cpu().numpy(), off_ref), "expert offsets differ"
    assert np.array_equal(srt.cpu().numpy(), srt_ref), "dispatch permutation differs"
    rows, counts = _prefill_rows(ids_ref, E, T, seed)
    y_ref, _, _ = O.moe_forward(x[rows], w, k, True, act, gs)
    stats = assert_moe_close(to_np(y)[rows], y_ref, act, f"prefill T={T}")
    print(f"prefill T={T}: {len(rows)} rows checked, expert load max/mean "
          f"{counts.max() / counts.mean():.1f}, {stats}", flush=True)
    return counts


@pytest.mark.parametrize("routing", ["uniform", "zipf"])
def test_moe_30b_prefill_4096(routing):
    """The 30B-A3B layer at 4096 tokens (the prefill headline workload),
    uniform and Zipf(1.1) routing; with Zipf the favourite expert fills
    about 32 m-tiles of the GEMM."""
    H, E, I, act, gs, T = 2048, 128, 768, "bfloat16", 64, 4096
    w = dict(_packed_weights(210, H, E, I, act))
    rng = np.random.default_rng(211)
    x = O.round_act(rng.standard_normal((T, H)), act)
    if routing == "zipf":
        x[:, :64] = 1.0
        w["router"] = _zipf_router(212, H, E, act)
    counts = _check_prefill(x, w, 8, act, gs, 213)
    if routing == "zipf":
        assert counts.max() >= 10 * counts.mean(), counts.max() / counts.mean()


def test_moe_235b_prefill_2048():
    """The 235B-A22B layer (hidden 4096, intermediate 1536) at 2048 tokens."""
    H, E, I, act, gs, T = 4096, 128, 1536, "bfloat16", 64, 2048
    w = _packed_weights(300, H, E, I, act)
    rng = np.random.default_rng(301)
    x = O.round_act(rng.standard_normal((T, H)), act)
    _check_prefill(x, w, 8, act, gs, 302)


@pytest.mark.parametrize("T", [32, 200])
def test_moe_graph_replay_matches_eager(T):
    """The fused forward captured in a HIP graph (as the benchmark times it)
    gives the eager result on every replay, with eager calls sharing the
    workspace in between.  T=32 takes the fused route-and-dispatch launch whose
    counters the router launch zeroes; T=200 the per-block dispatch."""
    x, w = _moe_case(900 + T, T, 2048, 128, 768, "bfloat16")
    moe = make_moe(w, "bfloat16", 64, 8, True, DEV)
    xt = to_act(x, "bfloat16", DEV)
    y_eager = moe(xt).clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        moe(xt)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_graph = moe(xt)
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_eager), f"replay {r} differs from the eager result"
        y_again = moe(xt)
        torch.cuda.synchronize()
        assert torch.equal(y_again, y_eager), f"eager call after replay {r} differs"
