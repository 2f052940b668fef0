"""Host-side parts of the reference's tensor, shape and nn tests
(tests/cpp/test_tensor.cpp, tests/python/test_shape.py, test_nn.py,
test_ffn.py): tensor factories and sizes, view metadata, Parameter and
Module registration.  No device compute; the device halves of these files
are in test_reference_suite_gpu.py."""
from __future__ import annotations

import numpy as np


def test_tensor_numel_sizes_and_factories(ag):
    # tests/cpp/test_tensor.cpp:12-35, :48-56
    t = ag.Tensor.empty([2, 3], ag.DType.Fp32)
    assert t.numel == 6
    assert ag.to_numpy(t).nbytes == 24
    h = ag.Tensor.empty([4, 4], ag.DType.Fp16)
    assert h.numel == 16 and ag.to_numpy(h).nbytes == 32
    s = ag.Tensor.empty([], ag.DType.Fp32)
    assert s.numel == 1 and s.shape == []
    np.testing.assert_array_equal(ag.to_numpy(ag.Tensor.zeros([4], ag.DType.Fp32)), np.zeros(4, np.float32))


def test_transpose_is_metadata_only(ag):
    # tests/python/test_shape.py:75-83
    x = ag.from_numpy(np.random.default_rng(10).standard_normal((2, 3, 4)).astype(np.float32))
    y = ag.transpose(x, 0, 2)
    assert y.shape == [4, 3, 2]
    assert y.strides == [x.strides[2], x.strides[1], x.strides[0]]
    assert y.is_contiguous() is False
    assert x.is_contiguous() is True
    assert y.storage_offset == x.storage_offset


def test_parameter_marks_requires_grad(ag):
    # tests/python/test_nn.py:17-21
    t = ag.from_numpy(np.zeros((2, 2), np.float32))
    assert t.requires_grad is False
    p = ag.nn.Parameter(t)
    assert p.tensor.requires_grad is True


def test_module_registers_parameters_and_submodules(ag):
    # tests/python/test_nn.py:24-42: own parameters first, then each child's
    nn = ag.nn

    class Inner(nn.Module):
        def __init__(self):
            super().__init__()
            self.w = nn.Parameter(ag.from_numpy(np.zeros((2, 2), np.float32)))

    class Outer(nn.Module):
        def __init__(self):
            super().__init__()
            self.a = nn.Parameter(ag.from_numpy(np.zeros((3,), np.float32)))
            self.inner = Inner()
            self.b = nn.Parameter(ag.from_numpy(np.zeros((4,), np.float32)))

    params = list(Outer().parameters())
    assert [p.tensor.shape for p in params] == [[3], [4], [2, 2]]


def test_linear_parameter_counts(ag):
    # tests/python/test_ffn.py:104-115
    assert len(list(ag.nn.Linear(4, 6, bias=True, rng=np.random.default_rng(0)).parameters())) == 2
    assert len(list(ag.nn.Linear(4, 6, bias=False, rng=np.random.default_rng(0)).parameters())) == 1


def test_lm_test_model_layout_and_init_draws(ag):
    """The Shakespeare test model (tests/lmutil.py) exposes the reference
    model's parameters in the reference's Module.parameters() order
    (python/shakespeare/scripts/model.py:8-57: tok_emb, pos_emb, per block
    ln1, attn qkv/out, ln2, fc1, fc2, then ln_f and the head), initialised by
    the same random draws in the same order."""
    import math

    import lmutil

    V, T, L, H, d = 11, 16, 2, 2, 8
    model = lmutil.GPT(V, T, L, H, d, rng=np.random.default_rng(5))
    got = [ag.to_numpy(p.tensor) for p in model.parameters()]
    rng = np.random.default_rng(5)

    def uni(fan_in, shape):
        b = math.sqrt(6.0 / fan_in)
        return rng.uniform(-b, b, size=shape).astype(np.float32)

    want = [rng.standard_normal((V, d)).astype(np.float32), rng.standard_normal((T, d)).astype(np.float32)]
    for _ in range(L):
        qkv, out = uni(d, (3 * d, d)), uni(d, (d, d))
        fc1, fc2 = uni(d, (4 * d, d)), uni(4 * d, (d, 4 * d))
        ones, zeros = np.ones(d, np.float32), np.zeros(d, np.float32)
        want += [ones, zeros, qkv, out, ones, zeros, fc1, np.zeros(4 * d, np.float32), fc2, zeros]
    want += [np.ones(d, np.float32), np.zeros(d, np.float32), uni(d, (V, d))]
    assert len(got) == len(want) == 2 + 10 * L + 3
    for i, (g, w) in enumerate(zip(got, want)):
        assert g.shape == w.shape, i
        np.testing.assert_array_equal(g, w)


def test_module_tree_order_train_and_to(ag):
    # parameters(): own parameters first, then each child's subtree in
    # registration order (aargrad/nn.py:27-31); re-assigning a registered name
    # keeps its position; train()/eval() reach every descendant
    nn = ag.nn

    def p(n):
        return nn.Parameter(ag.from_numpy(np.full(n, float(n), np.float32)))

    class Leaf(nn.Module):
        def __init__(self, n):
            super().__init__()
            self.w = p(n)

    class Mid(nn.Module):
        def __init__(self):
            super().__init__()
            self.first = Leaf(2)
            self.a = p(3)
            self.second = nn.Sequential(Leaf(4), nn.Dropout(0.5), Leaf(5))

    class Top(nn.Module):
        def __init__(self):
            super().__init__()
            self.x = p(1)
            self.mid = Mid()
            self.y = p(6)
            self.tail = Leaf(7)

    top = Top()
    assert [q.tensor.shape[0] for q in top.parameters()] == [1, 6, 3, 2, 4, 5, 7]
    top.x = p(9)  # replaces the entry in place
    assert [q.tensor.shape[0] for q in top.parameters()] == [9, 6, 3, 2, 4, 5, 7]
    top.note = "plain attribute"
    assert "note" not in top._parameters and "note" not in top._modules
    assert list(top.mid.second._modules) == ["layer_0", "layer_1", "layer_2"]
    top.eval()
    assert not top.mid.second.layer_1.training and not top.tail.training
    top.train()
    assert top.mid.second.layer_1.training
    moved = top.to(ag.Device.CPU)
    assert moved is top and all(q.tensor.requires_grad for q in top.parameters())
