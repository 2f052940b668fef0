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
