"""Ops called from several host threads at once.  Every op of aargrad._core
releases the GIL (as in the reference binding, cppsrc/python/binding.cpp:31),
so concurrent Python threads drive the caching allocator, the lazily created
device error slots and the autograd engine together.  All work is ordered on
one stream and every kernel is deterministic, so each thread's results must
equal the single-threaded ones bit for bit."""
from __future__ import annotations

import threading

import numpy as np
import pytest

from devutil import dev, host

pytestmark = pytest.mark.gpu
f32 = np.float32


def _work(gpu, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((96, 200)).astype(f32)
    b = rng.standard_normal((200, 72)).astype(f32)
    w = (1 + 0.1 * rng.standard_normal(72)).astype(f32)
    bb = (0.1 * rng.standard_normal(72)).astype(f32)
    q, k, v = (rng.standard_normal((2, 3, 70, 64)).astype(f32) for _ in range(3))
    ids = rng.integers(0, 65, (4, 9))
    out = []
    for _ in range(6):
        ta, tb = dev(gpu, a, True), dev(gpu, b, True)
        tw, tbb = dev(gpu, w, True), dev(gpu, bb, True)
        y = gpu.layernorm(gpu.matmul(ta, tb), tw, tbb, 1e-5)
        s = gpu.softmax(y)
        tq, tk, tv = dev(gpu, q, True), dev(gpu, k, True), dev(gpu, v, True)
        o = gpu.flash_attention(tq, tk, tv, True)
        loss = gpu.add(gpu.sum_all(gpu.mul(s, s)), gpu.sum_all(o))
        loss.backward()
        emb = gpu.embedding(dev(gpu, rng.standard_normal((65, 8)).astype(f32)),
                            gpu.from_numpy(ids).to(gpu.Device.CUDA))
        out.append([host(gpu, t) for t in (loss, ta.grad, tb.grad, tw.grad, tbb.grad, tq.grad, tk.grad, tv.grad)])
        out[-1].append(host(gpu, emb))
    return out


def test_concurrent_threads_match_serial(gpu):
    seeds = [11, 22, 33, 44]
    serial = {s: _work(gpu, s) for s in seeds}
    results, errors = {}, []

    def run(s):
        try:
            results[s] = _work(gpu, s)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=run, args=(s,)) for s in seeds]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    assert all(not t.is_alive() for t in threads)
    for s in seeds:
        for it_serial, it_par in zip(serial[s], results[s]):
            for x, y in zip(it_serial, it_par):
                np.testing.assert_array_equal(x, y)


def test_deferred_device_error_is_cleared_once_raised(gpu):
    # an out-of-range id is detected on the device and raised at the next host
    # synchronisation; the error word is then cleared, so later work is clean
    good = gpu.from_numpy(np.arange(8, dtype=np.int64) % 5).to(gpu.Device.CUDA)
    bad = gpu.from_numpy(np.array([0, 99], np.int64)).to(gpu.Device.CUDA)
    w = dev(gpu, np.ones((5, 4), f32))
    with pytest.raises(IndexError):
        host(gpu, gpu.embedding(w, bad))
    np.testing.assert_array_equal(host(gpu, gpu.embedding(w, good)), np.ones((8, 4), f32))


def test_forced_flash_plan_on_one_thread_leaves_another_on_the_default(gpu):
    """One thread runs the flash calls with a forced plan (128-query forward,
    128-key backward) through the C ABI's per-call plan entry points while
    another runs the same shape with the planner's choice (the paired 64-query
    and 64-key kernels at this shape).  The forced plan is an argument of the
    call, not library state, so each thread's results equal its own serial
    run bit for bit; the two plans themselves differ in rounding, so a plan
    leaking across threads would show."""
    from devutil import abi_flash

    rng = np.random.default_rng(17)
    q, k, v, do = (rng.standard_normal((8, 256, 64)).astype(f32) for _ in range(4))
    forced = abi_flash(q, k, v, do, True, query_block=128, key_block=128)
    default = abi_flash(q, k, v, do, True)
    assert any(not np.array_equal(a, b) for a, b in zip([forced[0]] + forced[2], [default[0]] + default[2]))
    results, errors = {"forced": [], "default": []}, []

    def run(name, kw):
        try:
            for _ in range(12):
                results[name].append(abi_flash(q, k, v, do, True, **kw))
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=run, args=("forced", {"query_block": 128, "key_block": 128})),
               threading.Thread(target=run, args=("default", {}))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    assert all(not t.is_alive() for t in threads)
    for name, ref in (("forced", forced), ("default", default)):
        assert len(results[name]) == 12
        for o, lse, grads in results[name]:
            np.testing.assert_array_equal(o, ref[0])
            np.testing.assert_array_equal(lse, ref[1])
            for g, r in zip(grads, ref[2]):
                np.testing.assert_array_equal(g, r)
