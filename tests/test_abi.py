"""The C ABI and the host-side mirror, without a GPU.

* libnvm_moe.so loads and exports every function declared in include/*.h;
* argument validation returns the documented status codes and messages
  before any device work (so it can be exercised on a CPU-only host);
* the Python mirror rejects CPU tensors and maps status codes to exceptions;
* the torch MLX-layout quantizer agrees with the oracle's.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _lib():
    from nano_vllm_metal_amd import _lib

    return _lib, _lib.load()


def test_library_exports_every_header_function():
    names = set()
    for h in HEADERS:
        names |= set(re.findall(r"^\s*(?:int|const char \*)\s*(nvm_\w+)\s*\(", h.read_text(), re.M))
    assert {"nvm_moe_forward", "nvm_paged_attention"} <= names and len(names) >= 14
    _, lib = _lib()
    for n in sorted(names):
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
    from nano_vllm_metal_amd._lib import SIGNATURES

    assert set(SIGNATURES) | {"nvm_abi_version", "nvm_last_error"} == names


def test_abi_version():
    L, lib = _lib()
    assert lib.nvm_abi_version() == L.ABI_VERSION == 2


def _err(lib) -> str:
    return lib.nvm_last_error().decode()


def test_workspace_sizes():
    L, lib = _lib()
    sz = ctypes.c_size_t()
    assert lib.nvm_moe_workspace_size(32, 2048, 768, 128, 8, ctypes.byref(sz)) == 0
    # partial logits + ids/scores + dispatch + h [N, I] + down [N, H]
    N = 32 * 8
    assert sz.value >= N * 768 * 2 + N * 2048 * 2
    assert lib.nvm_route_workspace_size(32, 2048, 128, ctypes.byref(sz)) == 0
    assert sz.value % 8 == 0 and sz.value >= 32 * 128 * 8
    assert lib.nvm_grouped_linear_workspace_size(100, 128, 64, 8, ctypes.byref(sz)) == 0
    assert lib.nvm_moe_workspace_size(32, 2048, 768, 128, 8, None) == L.NVM_ERR_INVALID


def _forward(lib, **kw):
    args = dict(x=1, T=4, H=2048, I=768, E=128, k=8, norm=1, gs=64, bits=4, dtype=1, y=1,
                regime=0, ws=1, ws_bytes=1 << 40)
    args.update(kw)
    p = [1] * 12  # weight pointers (never dereferenced: validation fails first)
    return lib.nvm_moe_forward(args["x"], args["T"], args["H"], args["I"], args["E"], args["k"],
                               args["norm"], args["gs"], args["bits"], args["dtype"], *p,
                               args["y"], None, None, args["regime"], args["ws"],
                               args["ws_bytes"], None)


@pytest.mark.parametrize("kw,code,msg", [
    ({"bits": 8}, -2, "bits must be 4"),
    ({"gs": 32}, -2, "group_size"),
    ({"dtype": 7}, -1, "dtype"),
    ({"H": 100}, -1, "hidden"),
    ({"I": 96}, -1, "intermediate"),
    ({"E": 1000}, -2, "experts"),
    ({"k": 0}, -1, "top_k"),
    ({"k": 200}, -1, "top_k"),
    ({"regime": 5}, -1, "regime"),
    ({"x": None}, -1, "null pointer"),
    ({"ws_bytes": 10}, -3, "workspace"),
])
def test_forward_validation(kw, code, msg):
    L, lib = _lib()
    assert _forward(lib, **kw) == code
    assert msg in _err(lib)


def test_forward_empty_batch_is_a_no_op():
    L, lib = _lib()
    assert _forward(lib, T=0) == 0


def test_noalloc_entry_point_validation():
    """nvm_moe_forward_noalloc: an empty batch is a no-op, and a batch whose
    workspace exceeds the static array is refused before any device work."""
    L, lib = _lib()
    cap = ctypes.c_size_t()
    assert lib.nvm_moe_scratch_bytes(ctypes.byref(cap)) == 0 and cap.value == 32 << 20
    p = [1] * 12

    def call(T):
        return lib.nvm_moe_forward_noalloc(1, T, 2048, 768, 128, 8, 1, 64, 4, 1, *p, 1, None,
                                           None, 0, None)

    assert call(0) == 0
    assert call(2048) == L.NVM_ERR_UNSUPPORTED and "static scratch" in _err(lib)
    assert lib.nvm_moe_forward_noalloc(1, -1, 2048, 768, 128, 8, 1, 64, 4, 1, *p, 1, None, None,
                                       0, None) == L.NVM_ERR_INVALID


def test_operands_beyond_32bit_offsets_are_refused():
    """The kernels address x and the weights through 32-bit buffer offsets:
    larger operands are refused instead of being read as zeros."""
    L, lib = _lib()
    T = 600_000  # 600000 x 2048 bf16 = 2.46 GB
    r = lib.nvm_moe_route(1, T, 2048, 1, 1, 1, 128, 64, 4, 8, 0, 1, None, 1, 1, 1, 1 << 40, None)
    assert r == L.NVM_ERR_UNSUPPORTED and "2 GiB" in _err(lib)
    r = lib.nvm_quantized_matmul(1, 1, 64, 4, 1, 1, 1, 1, T, 2048, 128, 1, None)
    assert r == L.NVM_ERR_UNSUPPORTED and "2 GiB" in _err(lib)
    # the whole block refuses such a batch before its first launch (the
    # routing would otherwise run and write the fp16 copy of x first)
    assert _forward(lib, T=T) == L.NVM_ERR_UNSUPPORTED and "2 GiB" in _err(lib)
    # h [T * k, I] beyond 2 GiB with x inside it
    assert _forward(lib, T=200_000) == L.NVM_ERR_UNSUPPORTED and "2 GiB" in _err(lib)


def test_quantized_matmul_validation():
    L, lib = _lib()
    # the reference requires transpose_b (quantized_matmul.cpp:56-58)
    r = lib.nvm_quantized_matmul(1, 1, 128, 4, 1, 1, 0, 1, 2, 128, 5, 1, None)
    assert r == L.NVM_ERR_UNSUPPORTED and "transposed" in _err(lib)
    r = lib.nvm_quantized_matmul(1, 1, 128, 4, 1, 1, 1, 1, 2, 100, 5, 1, None)
    assert r == L.NVM_ERR_INVALID and "divisible" in _err(lib)


def test_dispatch_and_route_validation():
    L, lib = _lib()
    assert lib.nvm_moe_dispatch(1, 10, 0, 1, 1, None, 0, None) == L.NVM_ERR_INVALID
    assert lib.nvm_moe_dispatch(1, 10, 4096, 1, 1, None, 0, None) == L.NVM_ERR_UNSUPPORTED
    # more than 4096 pairs sort over blocks and need the histogram workspace
    size = ctypes.c_size_t()
    assert lib.nvm_dispatch_workspace_size(4096, 128, ctypes.byref(size)) == 0 and size.value == 0
    assert lib.nvm_dispatch_workspace_size(32768, 128, ctypes.byref(size)) == 0
    assert size.value == 4 * 8 * 128
    assert lib.nvm_moe_dispatch(1, 32768, 128, 1, 1, None, 0, None) == L.NVM_ERR_WORKSPACE
    r = lib.nvm_moe_route_dispatch(1, 4, 2048, 1, 1, 1, 128, 64, 4, 8, 1, 1, None, 1, 1, 1, 1,
                                   None, 0, None)
    assert r == L.NVM_ERR_WORKSPACE
    r = lib.nvm_moe_route_dispatch(1, 4, 2048, 1, 1, 1, 128, 64, 4, 8, 1, 1, None, 1, 1, None, 1,
                                   1, 1 << 30, None)
    assert r == L.NVM_ERR_INVALID
    r = lib.nvm_moe_route(1, 4, 2048, 1, 1, 1, 128, 64, 4, 9, 0, 1, None, 1, 1, 1, 0, None)
    assert r == L.NVM_ERR_WORKSPACE
    r = lib.nvm_moe_route(1, 4, 2048, 1, 1, 1, 128, 64, 4, 129, 0, 1, None, 1, 1, 1, 1 << 30, None)
    assert r == L.NVM_ERR_INVALID


def test_check_maps_status_to_exceptions():
    L, lib = _lib()
    _forward(lib, bits=8)
    with pytest.raises(ValueError):
        L.check(L.NVM_ERR_UNSUPPORTED)
    with pytest.raises(RuntimeError):
        L.check(L.NVM_ERR_WORKSPACE)
    L.check(L.NVM_OK)


def test_python_mirror_rejects_cpu_tensors():
    from nano_vllm_metal_amd import Moe, QuantizedWeights, route_topk

    w = QuantizedWeights(torch.zeros(4, 2, dtype=torch.bfloat16), torch.zeros(4, 2, dtype=torch.bfloat16),
                         64, 4, torch.zeros(4, 16, dtype=torch.int32))
    with pytest.raises(ValueError, match="GPU only"):
        route_topk(torch.zeros(2, 128, dtype=torch.bfloat16), w, 2)
    moe = Moe(w, w, w, w, 2)
    with pytest.raises(ValueError, match="GPU only"):
        moe(torch.zeros(1, 2, 128, dtype=torch.bfloat16))


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import nano_vllm_metal_amd._lib as L

    monkeypatch.setattr(L, "_lib", None)
    monkeypatch.setenv("NVM_MOE_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        L.load()


@pytest.mark.parametrize("act", ["float16", "bfloat16"])
@pytest.mark.parametrize("gs", [64, 128])
def test_torch_quantizer_agrees_with_oracle(act, gs):
    from oracle import moe_oracle as O
    from nano_vllm_metal_amd import dequantize, quantize

    rng = np.random.default_rng(21)
    w = O.round_act(rng.standard_normal((24, 2 * gs)) * 0.02, act)
    dt = torch.float16 if act == "float16" else torch.bfloat16
    wq, s, b = quantize(torch.from_numpy(w.astype(np.float32)).to(dt), gs, 4)
    owq, os_, ob = O.quantize(w, gs, 4, act)
    # the torch path computes in float32, the oracle in float64: scales/biases
    # agree after rounding to act except in rare near-tie cases
    s_t = s.float().numpy().astype(np.float64)
    b_t = b.float().numpy().astype(np.float64)
    assert np.mean(s_t == os_) > 0.95 and np.mean(b_t == ob) > 0.95
    same = (s_t == os_) & (b_t == ob)
    codes_t = O.unpack_nibbles(wq.numpy().view(np.uint32))
    codes_o = O.unpack_nibbles(owq)
    rows = np.repeat(same, gs, axis=1)
    assert np.array_equal(codes_t[rows], codes_o[rows])
    # dequantisation of the torch layout equals the oracle's formula
    deq = dequantize(wq, s, b, gs).numpy().astype(np.float64)
    assert np.array_equal(deq, O.dequantize(wq.numpy().view(np.uint32), s_t, b_t, gs))


def _attn(lib, **kw):
    a = dict(q=1, N=64, L=1, D=128, kp=1, vp=1, P=8, ps=16, kv=1, ks=None, vs=None, bt=1, B=2,
             mp=4, lens=1, scale=0.1, causal=0, hkv=4, hq=32, odt=2, out=1, ws=1,
             ws_bytes=1 << 40)
    a.update(kw)
    return lib.nvm_paged_attention(a["q"], a["N"], a["L"], a["D"], a["kp"], a["vp"], a["P"],
                                   a["ps"], a["kv"], a["ks"], a["vs"], a["bt"], a["B"], a["mp"],
                                   a["lens"], a["scale"], a["causal"], a["hkv"], a["hq"],
                                   a["odt"], a["out"], a["ws"], a["ws_bytes"], None)


@pytest.mark.parametrize("kw,code,msg", [
    ({"hq": 30}, -1, "divisible by num_kv_heads"),
    ({"N": 65}, -1, "divisible by num_heads"),
    ({"B": 3}, -1, "batch size"),
    ({"kv": 5}, -1, "kv dtype"),
    ({"D": 512}, -2, "head dimension"),
    ({"kv": 3}, -1, "key_scales and value_scales"),
    ({"q": None}, -1, "null pointer"),
    ({"ws": None, "mp": 80}, -3, "workspace"),
    ({"P": 1 << 20, "ps": 64}, -2, "2 GiB"),
    ({"odt": 3}, -1, "out dtype"),
])
def test_paged_attention_validation(kw, code, msg):
    """Argument checks of nvm_paged_attention (the reference's paged_attention
    op checks, metal/src/paged_attention.cpp:21-63) return before device work."""
    _, lib = _lib()
    assert _attn(lib, **kw) == code
    assert msg in _err(lib)


def _causal(lib, **kw):
    a = dict(q=1, k=1, v=1, B=2, L=16, hq=32, hkv=4, D=128, scale=0.088, dt=1, odt=1, out=1)
    a.update(kw)
    return lib.nvm_causal_attention(a["q"], a["k"], a["v"], a["B"], a["L"], a["hq"], a["hkv"],
                                    a["D"], a["scale"], a["dt"], a["odt"], a["out"], None)


@pytest.mark.parametrize("kw,code,msg", [
    ({"scale": 0.0}, -2, "scale must be positive"),
    ({"scale": -0.1}, -2, "scale must be positive"),
    ({"scale": float("nan")}, -2, "scale must be positive"),
    ({"scale": float("inf")}, -2, "scale must be positive"),
    ({"D": 96}, -2, "head dim"),
    ({"hq": 24, "hkv": 8}, -2, "query heads per kv head"),
    ({"hq": 30}, -1, "bad shape"),
    ({"dt": 7}, -1, "dtype must be f16 or bf16"),
    ({"q": None}, -1, "null pointer"),
])
def test_causal_attention_validation(kw, code, msg):
    """Argument checks of nvm_causal_attention return before device work.  The
    kernel's softmax takes the maximum of the raw scores and scales it, so the
    scale must be positive (the model passes head_dim ** -0.5)."""
    _, lib = _lib()
    assert _causal(lib, **kw) == code
    assert msg in _err(lib)


def test_paged_attention_workspace_size():
    _, lib = _lib()
    sz = ctypes.c_size_t()
    # decode, 32 requests x 4 kv heads, 1280 positions: the context is split
    assert lib.nvm_paged_attention_workspace_size(32 * 32, 1, 128, 80, 16, 1, 4, 32,
                                                  ctypes.byref(sz)) == 0
    assert sz.value >= 32 * 32 * 2 * 128 * 4
    # one row kernel (multi-query): no workspace
    assert lib.nvm_paged_attention_workspace_size(32 * 32, 4, 128, 80, 16, 1, 4, 32,
                                                  ctypes.byref(sz)) == 0
    assert sz.value == 0


@pytest.mark.parametrize("call,code,msg", [
    (lambda lib: lib.nvm_residual_rms_norm(1, 1, 1, 4, 2047, 1e-6, 1, 1, 1, None), -1, "bad shape"),
    (lambda lib: lib.nvm_residual_rms_norm(1, 1, 1, 4, 16384, 1e-6, 1, 1, 1, None), -2, "at most"),
    (lambda lib: lib.nvm_residual_rms_norm(1, 1, 1, 4, 2048, 1e-6, 7, 1, 1, None), -1, "dtype"),
    (lambda lib: lib.nvm_residual_rms_norm(1, 1, 1, 4, 2048, 1e-6, 1, None, 1, None), -1, "null"),
    (lambda lib: lib.nvm_qk_norm_rope_store(1, 4, 32, 4, 130, 1, 1, 1e-6, 1, 1, 1, 100, 1, 1, 1, 1,
                                            8, 16, 1, 1, None, None, None), -2, "multiple of 4"),
    (lambda lib: lib.nvm_qk_norm_rope_store(1, 4, 32, 4, 128, 1, 1, 1e-6, 1, 1, 1, 100, 1, 1, 1, 1,
                                            8, 16, 1, None, None, None, None), -1, "null"),
    (lambda lib: lib.nvm_moe_forward_residual_norm(1, 4, 2052, 768, 128, 8, 1, 64, 4, 1,
                                                   *([1] * 12), 1, 1, 1e-6, 1, 1, 0, 1, 1 << 40,
                                                   None), -2, "multiple of 8"),
    (lambda lib: lib.nvm_moe_forward_residual_norm(1, 4, 2048, 768, 128, 8, 1, 64, 4, 1,
                                                   *([1] * 12), None, 1, 1e-6, 1, 1, 0, 1,
                                                   1 << 40, None), -1, "null pointer"),
    (lambda lib: lib.nvm_moe_forward_residual_norm(1, 4, 2048, 768, 128, 8, 1, 64, 4, 1,
                                                   *([1] * 12), 24, 16, 1e-6, 16, 16, 0, 1,
                                                   1 << 40, None), -1, "16-byte aligned"),
])
def test_model_ops_validation(call, code, msg):
    """nvm_residual_rms_norm / nvm_qk_norm_rope_store reject bad arguments
    before any device work."""
    _, lib = _lib()
    assert call(lib) == code
    assert msg in _err(lib)


def test_forward_stage_validation():
    """nvm_moe_forward_stage checks its stage index and then validates as
    nvm_moe_forward does, before any device work."""
    L, lib = _lib()
    p = [1] * 12

    def call(stage, T=4, bits=4):
        return lib.nvm_moe_forward_stage(stage, 1, T, 2048, 768, 128, 8, 1, 64, bits, 1, *p, 1,
                                         None, None, 0, 1, 1 << 40, None)

    assert call(6) == L.NVM_ERR_INVALID and "stage" in _err(lib)
    assert call(-1) == L.NVM_ERR_INVALID
    assert call(1, bits=8) == L.NVM_ERR_UNSUPPORTED and "bits" in _err(lib)
    assert call(0, T=0) == 0
    assert call(2, T=600_000) == L.NVM_ERR_UNSUPPORTED and "2 GiB" in _err(lib)


def test_forward_plan(monkeypatch):
    """nvm_moe_forward_plan: one launch for both decode products at the
    30B-A3B shape from one routed row per expert on average up to 64 tokens
    (regime auto or decode), else the separate products; the overrides
    NVM_FUSED_DOWN and NVM_GEMV_STATIC=0 apply; no device work."""
    import ctypes

    L, lib = _lib()
    monkeypatch.delenv("NVM_FUSED_DOWN", raising=False)
    monkeypatch.delenv("NVM_GEMV_STATIC", raising=False)

    def plan(T, H=2048, I=768, E=128, k=8, gs=64, regime=0):
        out = ctypes.c_int(-1)
        assert lib.nvm_moe_forward_plan(T, H, I, E, k, gs, regime, ctypes.byref(out)) == 0
        return out.value

    assert [plan(T) for T in (1, 8, 15, 16, 32, 64, 65, 4096)] == [0, 0, 0, 1, 1, 1, 0, 0]
    assert plan(32, regime=1) == 1 and plan(32, regime=2) == 0
    assert plan(32, H=4096, I=1536) == 0 and plan(32, gs=128) == 0
    monkeypatch.setenv("NVM_FUSED_DOWN", "1")
    assert plan(1) == 1 and plan(65) == 0
    monkeypatch.setenv("NVM_FUSED_DOWN", "0")
    assert plan(32) == 0
    monkeypatch.delenv("NVM_FUSED_DOWN")
    monkeypatch.setenv("NVM_GEMV_STATIC", "0")
    assert plan(32) == 0
    assert lib.nvm_moe_forward_plan(32, 2048, 768, 128, 8, 64, 0, None) == L.NVM_ERR_INVALID
