"""CPU-side checks of the boundary: the C-ABI library loads and exports every
entry point declared in include/aar_hip.h, and the host layer (aargrad._core)
keeps the reference API, validation errors and view semantics.  No kernel is
launched here (no GPU in this container)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "aar_hip.h"
LIB = REPO / "aar-vlm_amd" / "aargrad" / "libaar_hip.so"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(aar_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_dispatch_surface():
    syms = declared_symbols()
    for s in ("aar_gemm_f32", "aar_softmax_fwd_f32", "aar_softmax_bwd_f32", "aar_layernorm_fwd_f32",
              "aar_layernorm_bwd_f32", "aar_flash_fwd_f32", "aar_flash_bwd_f32", "aar_add_f32",
              "aar_malloc", "aar_free", "aar_memcpy", "aar_memset_zero", "aar_synchronize",
              "aar_error_string"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(LIB))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_error_strings():
    lib = ctypes.CDLL(str(LIB))
    lib.aar_error_string.restype = ctypes.c_char_p
    assert lib.aar_error_string(0) == b"ok"
    assert b"invalid" in lib.aar_error_string(-1)
    assert b"workspace" in lib.aar_error_string(-2)
    assert b"memory" in lib.aar_error_string(-4)


def test_abi_validates_before_touching_the_device():
    lib = ctypes.CDLL(str(LIB))
    vp = ctypes.c_void_p
    i64 = ctypes.c_int64
    lib.aar_gemm_f32.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, ctypes.c_size_t, vp]
    assert lib.aar_gemm_f32(7, 2, 2, 2, None, None, None, None, 0, None) == -1  # bad op
    assert lib.aar_gemm_f32(0, -1, 2, 2, None, None, None, None, 0, None) == -1
    assert lib.aar_gemm_f32(0, 0, 2, 2, None, None, None, None, 0, None) == 0  # empty is a no-op
    lib.aar_gemm_f32_bias.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
    assert lib.aar_gemm_f32_bias(3, 2, 2, 2, None, None, None, None, None, 0, None) == -1  # bad op
    assert lib.aar_gemm_f32_bias(1, 2, 2, 2, None, None, None, None, None, 0, None) == -1  # no bias
    assert lib.aar_gemm_f32_bias(1, 2, 0, 2, None, None, None, None, None, 0, None) == 0  # empty output
    # fused relu epilogues: bias + relu on the NT product only, the relu mask on the NN product only
    for f in (lib.aar_gemm_f32_bias_relu, lib.aar_gemm_f32_relu_mask):
        f.argtypes = lib.aar_gemm_f32_bias.argtypes
    x = ctypes.c_void_p(16)  # never dereferenced: every call below returns before any device work
    assert lib.aar_gemm_f32_bias_relu(1, 2, 2, 2, None, None, None, None, None, 0, None) == -1  # no bias
    assert lib.aar_gemm_f32_bias_relu(0, 2, 2, 2, None, None, x, None, None, 0, None) == -3  # NN
    assert lib.aar_gemm_f32_bias_relu(1, 2, 2, 0, None, None, x, None, None, 0, None) == -3  # K == 0
    assert lib.aar_gemm_f32_bias_relu(1, 0, 2, 2, None, None, None, None, None, 0, None) == 0  # empty output
    assert lib.aar_gemm_f32_relu_mask(0, 2, 2, 2, None, None, None, None, None, 0, None) == -1  # no mask
    assert lib.aar_gemm_f32_relu_mask(1, 2, 2, 2, None, None, x, None, None, 0, None) == -3  # NT
    assert lib.aar_gemm_f32_relu_mask(3, 2, 2, 2, None, None, x, None, None, 0, None) == -1  # bad op
    # the mask as bits: bias + relu + bits on NT only; the masked NN product with column sums needs
    # bits, column sums and a row count of 64-row colsum chunks
    lib.aar_gemm_f32_bias_relu_bits.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, vp,
                                                ctypes.c_size_t, vp]
    lib.aar_gemm_f32_mask_bits_colsum.argtypes = lib.aar_gemm_f32_bias_relu_bits.argtypes
    lib.aar_gemm_f32_mask_bits_colsum_workspace_bytes.restype = ctypes.c_size_t
    lib.aar_gemm_f32_mask_bits_colsum_workspace_bytes.argtypes = [i64, i64]
    assert lib.aar_gemm_f32_bias_relu_bits(1, 2, 2, 2, None, None, x, None, None, None, 0, None) == -1  # no bits
    assert lib.aar_gemm_f32_bias_relu_bits(1, 2, 2, 2, None, None, None, None, x, None, 0, None) == -1  # no bias
    assert lib.aar_gemm_f32_bias_relu_bits(0, 2, 2, 2, None, None, x, None, x, None, 0, None) == -3  # NN
    assert lib.aar_gemm_f32_bias_relu_bits(1, 0, 2, 2, None, None, None, None, None, None, 0, None) == 0
    assert lib.aar_gemm_f32_mask_bits_colsum(0, 64, 2, 2, None, None, x, None, None, None, 0, None) == -1
    assert lib.aar_gemm_f32_mask_bits_colsum(0, 64, 2, 2, None, None, None, None, x, None, 0, None) == -1
    assert lib.aar_gemm_f32_mask_bits_colsum(1, 64, 2, 2, None, None, x, None, x, None, 0, None) == -3  # NT
    assert lib.aar_gemm_f32_mask_bits_colsum(0, 100, 2, 2, None, None, x, None, x, None, 0, None) == -3
    assert lib.aar_gemm_f32_mask_bits_colsum(0, 64, 2, 0, None, None, x, None, x, None, 0, None) == -3  # K = 0
    assert lib.aar_gemm_f32_mask_bits_colsum(0, 64, 0, 2, None, None, None, None, None, None, 0, None) == 0
    assert lib.aar_gemm_f32_mask_bits_colsum_workspace_bytes(16384, 1536) == 256 * 1536 * 4
    assert lib.aar_gemm_f32_mask_bits_colsum_workspace_bytes(0, 1536) == 0
    # weight + bias gradients in one TN pass: TN only, whole 64-row colsum chunks
    lib.aar_gemm_f32_colsum_a.argtypes = [ctypes.c_int, i64, i64, i64, vp, vp, vp, vp, vp, ctypes.c_size_t, vp]
    lib.aar_gemm_f32_colsum_a_workspace_bytes.restype = ctypes.c_size_t
    lib.aar_gemm_f32_colsum_a_workspace_bytes.argtypes = [ctypes.c_int, i64, i64, i64]
    assert lib.aar_gemm_f32_colsum_a(2, 2, 2, 64, None, None, None, None, None, 0, None) == -1  # no colsum
    assert lib.aar_gemm_f32_colsum_a(0, 2, 2, 64, None, None, None, x, None, 0, None) == -3  # NN
    assert lib.aar_gemm_f32_colsum_a(2, 2, 2, 100, None, None, None, x, None, 0, None) == -3  # K not 64-row chunks
    assert lib.aar_gemm_f32_colsum_a(2, 0, 2, 64, None, None, None, None, None, 0, None) == 0  # empty
    assert lib.aar_gemm_f32_colsum_a_workspace_bytes(0, 384, 1536, 16384) == 0
    assert lib.aar_gemm_f32_colsum_a_workspace_bytes(2, 384, 1536, 16384) >= 256 * 384 * 4
    assert lib.aar_gemm_f32_bias(1, 2, 2, 0, None, None, 16, None, None, 0, None) == -3  # K = 0: not a product
    lib.aar_softmax_fwd_f32.argtypes = [vp, vp, i64, i64, vp]
    assert lib.aar_softmax_fwd_f32(None, None, 4, 0, None) == -1
    lib.aar_flash_fwd_f32.argtypes = [vp] * 5 + [i64, i64, i64, ctypes.c_int, ctypes.c_float, vp]
    assert lib.aar_flash_fwd_f32(None, None, None, None, None, 1, 8, 256, 1, 1.0, None) == -1  # d > 128
    lib.aar_flash_bwd_workspace_bytes.restype = ctypes.c_size_t
    lib.aar_flash_bwd_workspace_bytes.argtypes = [i64, i64, i64]
    assert lib.aar_flash_bwd_workspace_bytes(96, 4096, 64) == 96 * 4096 * 4
    # stored-dS workspace: D rows (256-byte padded) + one 32x32 tile per pair with work
    lib.aar_flash_bwd_fast_workspace_bytes.restype = ctypes.c_size_t
    lib.aar_flash_bwd_fast_workspace_bytes.argtypes = [i64, i64, i64, ctypes.c_int]
    d_rows = (96 * 4096 * 4 + 255) // 256 * 256
    assert lib.aar_flash_bwd_fast_workspace_bytes(96, 4096, 64, 1) == d_rows + 96 * (128 * 129 // 2) * 4096
    assert lib.aar_flash_bwd_fast_workspace_bytes(96, 4096, 64, 0) == d_rows + 96 * 128 * 128 * 4096
    assert lib.aar_flash_bwd_fast_workspace_bytes(3, 45, 64, 1) == 768 + 3 * 3 * 4096  # ragged T: 540 B of D rows
    # forward split partials: S = nqb/2 blocks x 2 halves x 128 rows, O rows of
    # the padded head dim (256-byte aligned) then one log2-sum-exp per row
    lib.aar_flash_fwd_workspace_bytes.restype = ctypes.c_size_t
    lib.aar_flash_fwd_workspace_bytes.argtypes = [i64, i64, i64, ctypes.c_int]
    rows = 96 * 4 * 2 * 128
    assert lib.aar_flash_fwd_workspace_bytes(96, 1024, 64, 1) == rows * 64 * 4 + rows * 4
    assert lib.aar_flash_fwd_workspace_bytes(2, 300, 30, 1) == 2 * 1 * 2 * 128 * (32 + 1) * 4
    assert lib.aar_flash_fwd_workspace_bytes(96, 1024, 64, 0) == 0  # only the causal forward splits
    assert lib.aar_flash_fwd_workspace_bytes(96, 4096, 64, 1) == 0  # 3072 workgroups: several rounds, no split
    assert lib.aar_flash_fwd_workspace_bytes(3, 128, 64, 1) == 0  # one query block
    assert lib.aar_flash_fwd_workspace_bytes(3, 100, 200, 1) == 0  # d > 128
    assert lib.aar_flash_bwd_fast_workspace_bytes(1 << 24, 1 << 24, 64, 0) == 2 ** 64 - 1  # saturates
    # token windows, dropout, causal mask: argument checks before any launch
    lib.aar_token_windows_i64.argtypes = [vp, i64, vp, i64, i64, vp, vp, vp, vp]
    assert lib.aar_token_windows_i64(None, 10, None, 2, 0, None, None, None, None) == -1  # seq_len 0
    assert lib.aar_token_windows_i64(None, 10, None, 0, 4, None, None, None, None) == 0  # empty batch
    lib.aar_dropout_f32.argtypes = [vp, vp, vp, i64, ctypes.c_float, ctypes.c_uint64, vp]
    assert lib.aar_dropout_f32(None, None, None, 4, 1.0, 0, None) == -1  # p outside [0, 1)
    assert lib.aar_dropout_f32(None, None, None, 0, 0.5, 0, None) == 0
    lib.aar_causal_mask_f32.argtypes = [vp, vp, i64, i64, ctypes.c_float, vp]
    assert lib.aar_causal_mask_f32(None, None, -1, 4, 0.0, None) == -1
    # multi-tensor optimizer updates: list and size checks before any launch
    pp = ctypes.POINTER(vp)
    lib.aar_scaled_add_multi_f32.argtypes = [ctypes.c_int, pp, pp, ctypes.POINTER(i64), ctypes.c_float, vp]
    assert lib.aar_scaled_add_multi_f32(-1, None, None, None, 1.0, None) == -1
    assert lib.aar_scaled_add_multi_f32(0, None, None, None, 1.0, None) == 0
    assert lib.aar_scaled_add_multi_f32(2, None, None, None, 1.0, None) == -1
    ptrs = (vp * 1)(None)
    sizes = (i64 * 1)(-3)
    assert lib.aar_scaled_add_multi_f32(1, ptrs, ptrs, sizes, 1.0, None) == -1  # negative size
    sizes[0] = 8
    assert lib.aar_scaled_add_multi_f32(1, ptrs, ptrs, sizes, 1.0, None) == -1  # null pointer with n > 0
    lib.aar_adamw_multi_f32.argtypes = [ctypes.c_int, pp, pp, pp, pp, ctypes.POINTER(i64)] + [ctypes.c_float] * 7 + [vp]
    assert lib.aar_adamw_multi_f32(1, ptrs, ptrs, ptrs, ptrs, sizes, *([0.1] * 7), None) == -1
    sizes[0] = 0
    assert lib.aar_adamw_multi_f32(1, ptrs, ptrs, ptrs, ptrs, sizes, *([0.1] * 7), None) == 0  # all empty: no launch


def test_gemm_workspace_query_buys_the_unlimited_plan():
    """A caller that passes the bytes aar_gemm_f32_workspace_bytes reports
    gets the plan an unlimited workspace gets (planning only, no launch; the
    CU count is the device's, 256 without one).  Split counts the planner
    asks for can shrink when the K chunk is rounded to the tile depth
    (384 x 384 x 16384 TN: 28 asked, 27 real); the plan's workspace is the
    real count's."""
    lib = ctypes.CDLL(str(LIB))
    i64, sz, ip = ctypes.c_int64, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int)
    lib.aar_gemm_f32_plan.argtypes = [ctypes.c_int, i64, i64, i64, sz, ip, ip]
    lib.aar_gemm_f32_workspace_bytes.restype = sz
    lib.aar_gemm_f32_workspace_bytes.argtypes = [ctypes.c_int, i64, i64, i64]

    def plan(op, M, N, K, ws):
        cfg, sp = ctypes.c_int(), ctypes.c_int()
        assert lib.aar_gemm_f32_plan(op, M, N, K, ws, ctypes.byref(cfg), ctypes.byref(sp)) == 0
        return cfg.value, sp.value

    checked = split = 0
    dims = (64, 65, 128, 384, 1000, 1152, 1536, 4096)
    for op in (0, 1, 2):
        for M in dims:
            for N in dims:
                for K in (384, 4096, 16384, 65536):
                    ws = lib.aar_gemm_f32_workspace_bytes(op, M, N, K)
                    want = plan(op, M, N, K, 1 << 40)
                    assert plan(op, M, N, K, ws) == want, (op, M, N, K, ws)
                    checked += 1
                    split += want[1] > 1
    assert split > 50, (checked, split)
    assert plan(2, 384, 384, 16384, lib.aar_gemm_f32_workspace_bytes(2, 384, 384, 16384))[1] == 27


def test_core_exports_reference_api(ag):
    for name in ("Tensor", "DType", "Device", "from_numpy", "to_numpy", "add", "sub", "mul", "relu",
                 "gelu", "sum_all", "add_bias", "scale", "matmul", "matmul_a_bt", "matmul_at_b",
                 "softmax", "layernorm", "apply_causal_mask", "reshape", "transpose", "slice",
                 "squeeze", "unsqueeze", "contiguous", "bmm", "bmm_a_bt", "bmm_at_b", "embedding",
                 "cross_entropy", "dropout", "manual_seed", "scaled_add_inplace", "adamw_step",
                 "flash_attention", "cuda_synchronize"):
        assert hasattr(ag, name), name
    assert ag.Device.CUDA is not None and ag.DType.Fp32 is not None


def test_factories_and_numpy_round_trip(ag):
    # tests/python/test_smoke.py:23-42 (host-side plumbing)
    z = ag.Tensor.zeros([2, 3], ag.DType.Fp32)
    o = ag.Tensor.ones([2, 3], ag.DType.Fp32)
    assert z.numel == 6 and z.shape == [2, 3] and z.strides == [3, 1]
    np.testing.assert_array_equal(ag.to_numpy(z), np.zeros((2, 3), np.float32))
    np.testing.assert_array_equal(ag.to_numpy(o), np.ones((2, 3), np.float32))
    x = np.arange(6, dtype=np.float16).reshape(2, 3)
    t = ag.from_numpy(x)
    assert t.dtype == ag.DType.Fp16
    np.testing.assert_array_equal(ag.to_numpy(t), x)
    assert repr(ag.from_numpy(np.zeros((2, 3), np.float32))) == "Tensor(shape=[2, 3], dtype=Fp32, device=CPU)"


def test_reshape_shape_rules(ag):
    # the reference reshape's rules and messages (cppsrc/ops/shape.cpp:15-44):
    # one inferred -1 at most, no other negative extent, the first offending
    # entry from the left picks the message
    t = ag.from_numpy(np.arange(24, dtype=np.float32))
    assert ag.reshape(t, [2, -1, 3]).shape == [2, 4, 3]
    assert ag.reshape(t, [24]).shape == [24]
    assert ag.reshape(ag.from_numpy(np.zeros((0, 3), np.float32)), [3, 0]).shape == [3, 0]
    for shape, msg in (([5, -1], "cannot infer"), ([0, -1], "cannot infer"), ([5, 5], "numel mismatch"),
                       ([-1, -1], "at most one -1"), ([-2, 12], "negative dim other than -1"),
                       ([-1, -1, -2], "at most one -1"), ([-2, -1, -1], "negative dim other than -1")):
        with pytest.raises(ValueError, match=msg):
            ag.reshape(t, shape)


def test_views_on_host(ag):
    a = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    t = ag.from_numpy(a)
    tr = ag.transpose(t, 0, 2)
    assert not tr.is_contiguous() and tr.shape == [4, 3, 2]
    np.testing.assert_array_equal(ag.to_numpy(tr), a.transpose(2, 1, 0))
    s = ag.slice(t, 1, 1, 3)
    np.testing.assert_array_equal(ag.to_numpy(s), a[:, 1:3])
    np.testing.assert_array_equal(ag.to_numpy(ag.reshape(t, [-1, 4])), a.reshape(-1, 4))
    np.testing.assert_array_equal(ag.to_numpy(ag.unsqueeze(t, 0)), a[None])
    np.testing.assert_array_equal(ag.to_numpy(ag.squeeze(ag.unsqueeze(t, 3), 3)), a)
    with pytest.raises(ValueError):
        ag.reshape(t, [5, -1])
    with pytest.raises(ValueError):
        ag.transpose(t, 0, 3)
    with pytest.raises(ValueError):
        ag.slice(t, 1, 2, 2)
    with pytest.raises(ValueError):
        ag.squeeze(t, 0)


def test_validation_errors_match_reference(ag):
    # std::invalid_argument -> ValueError, as in the reference binding
    f = lambda *s: ag.from_numpy(np.zeros(s, np.float32))  # noqa: E731
    with pytest.raises(ValueError, match="inner dimensions mismatch"):
        ag.matmul(f(2, 3), f(4, 2))  # tests/cpp/test_matmul.cpp:52-56
    with pytest.raises(ValueError, match="dtype mismatch"):
        ag.matmul(f(2, 2), ag.from_numpy(np.zeros((2, 2), np.float16)))
    with pytest.raises(ValueError):
        ag.matmul_a_bt(f(2, 3), f(2, 4))
    with pytest.raises(ValueError):
        ag.matmul_at_b(f(3, 2), f(4, 2))
    with pytest.raises(ValueError):
        ag.softmax(ag.Tensor.empty([], ag.DType.Fp32))  # tests/cpp/test_softmax.cpp:67-70
    with pytest.raises(ValueError):
        ag.layernorm(f(4), f(3), f(4))  # tests/cpp/test_layernorm.cpp:100-105
    with pytest.raises(ValueError, match="eps"):
        ag.layernorm(f(2, 4), f(4), f(4), 0.0)
    with pytest.raises(ValueError, match="share shape"):
        ag.flash_attention(f(1, 2, 4, 8), f(1, 2, 4, 8), f(1, 2, 5, 8), True)
    with pytest.raises(ValueError, match="at least 3 dims"):
        ag.flash_attention(f(4, 8), f(4, 8), f(4, 8), True)
    # the fused linear keeps the messages of matmul_a_bt and add_bias
    with pytest.raises(ValueError, match="contraction dim mismatch"):
        ag._core._linear(f(2, 3), f(4, 2), f(4))
    with pytest.raises(ValueError, match="bias must be 1-D"):
        ag._core._linear(f(2, 3), f(4, 3), f(1, 4))
    with pytest.raises(ValueError, match="bias size must match"):
        ag._core._linear(f(2, 3), f(4, 3), f(5))
    # the fused MLP raises what the composition linear -> relu -> linear raises
    with pytest.raises(ValueError, match="contraction dim mismatch"):
        ag._core._mlp_relu(f(2, 3), f(4, 2), f(4), f(5, 4), f(5))
    with pytest.raises(ValueError, match="bias size must match"):
        ag._core._mlp_relu(f(2, 3), f(4, 3), f(3), f(5, 4), f(5))


def test_host_compute_fails_loudly(ag):
    f = lambda *s: ag.from_numpy(np.zeros(s, np.float32))  # noqa: E731
    for call in (lambda: ag.matmul(f(2, 3), f(3, 2)),
                 lambda: ag.softmax(f(2, 3)),
                 lambda: ag.layernorm(f(2, 3), f(3), f(3)),
                 lambda: ag.flash_attention(f(1, 4, 8), f(1, 4, 8), f(1, 4, 8), True),
                 lambda: ag.add(f(3), f(3)),
                 lambda: ag.sum_all(f(3)),
                 lambda: ag._core._linear(f(2, 3), f(4, 3), f(4)),
                 lambda: ag._core._mlp_relu(f(2, 3), f(4, 3), f(4), f(5, 4), f(5))):
        with pytest.raises(RuntimeError, match="GPU only"):
            call()


def test_backward_arity_and_shape_errors(ag):
    x = ag.from_numpy(np.zeros((3,), np.float32), requires_grad=True)
    y = ag.reshape(x, [3, 1])
    with pytest.raises(RuntimeError, match="scalar"):
        y.backward()
    with pytest.raises(RuntimeError, match="shape mismatch"):
        y.backward(ag.from_numpy(np.ones((3,), np.float32)))
    # a view-only graph needs no arithmetic: the seed flows back to the leaf
    y.backward(ag.from_numpy(np.arange(3, dtype=np.float32).reshape(3, 1)))
    np.testing.assert_array_equal(ag.to_numpy(x.grad), np.arange(3, dtype=np.float32))
    x.zero_grad()
    assert x.grad is None
    with pytest.raises(RuntimeError, match="non-leaf"):
        y.requires_grad = True


def test_gemm_plan_substitutions():
    """The planner's substitutions (planning only, 256 CUs without a device):
    configuration 16 (the 128 x 192 tile as 8 waves) for NN/NT plans on 8
    over at most one tile per CU and for NT/TN plans on 6 whose 128 x 192
    grid is three or more whole rounds; configuration 15 (6 with a deeper
    ring) for other unsplit plans on 6 of three or more tiles per CU."""
    lib = ctypes.CDLL(str(LIB))
    i64, sz, ip = ctypes.c_int64, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int)
    lib.aar_gemm_f32_plan.argtypes = [ctypes.c_int, i64, i64, i64, sz, ip, ip]

    def cfg(op, M, N, K):
        c, s = ctypes.c_int(), ctypes.c_int()
        assert lib.aar_gemm_f32_plan(op, M, N, K, 1 << 30, ctypes.byref(c), ctypes.byref(s)) == 0
        return c.value

    NN, NT, TN = 0, 1, 2
    for K in (384, 1152, 1536):  # the GPT step's one-tile-per-CU products
        assert cfg(NN, 16384, 384, K) == 16 and cfg(NT, 16384, 384, K) == 16
    assert cfg(TN, 16384, 384, 384) == 8  # TN keeps 8
    assert cfg(NT, 16384, 1152, 384) == 16 and cfg(TN, 16384, 1152, 384) == 16  # 3 whole rounds
    assert cfg(NT, 24576, 1152, 384) != 16  # 4.5 rounds: a partial last round
    assert cfg(NT, 16384, 1536, 384) == 8  # two tiles per CU: 8 itself
    # unsplit plans on 6 of three or more 64 x 128 tiles per CU whose 128 x 192 grid is not whole rounds
    assert cfg(NN, 384, 16384, 384) == 15 and cfg(NT, 16384, 640, 384) == 15 and cfg(TN, 16384, 640, 1024) == 15
