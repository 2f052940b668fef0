"""Device side of the data formats: the HBM-resident token loader gives the
reference DataLoader's batches exactly (int64, bit-exact); window errors are
raised; checkpoints round-trip through the device bit-exactly; and the
checkpoint the reference ships loads and runs, matching the oracle's forward
of the same model (tolerance 1e-4, both metrics)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import lmutil
from aargrad import checkpoint as ck
from aargrad import data as D
from conftest import assert_close
from devutil import dev, host

pytestmark = pytest.mark.gpu
FIX = Path(__file__).resolve().parent / "golden" / "shakespeare"


def _i64(gpu, t):
    return gpu.to_numpy(t.to(gpu.Device.CPU))


@pytest.mark.parametrize("T,bs,shuffle,drop_last", [(32, 16, True, True), (256, 8, True, True),
                                                     (1, 3, False, False), (100, 64, False, True)])
def test_device_loader_equals_reference_loader(gpu, T, bs, shuffle, drop_last):
    ids = D.read_tokens(FIX / "val_head.bin")
    ref = D.DataLoader(D.TokenWindowDataset(ids, T), bs, shuffle=shuffle, drop_last=drop_last, seed=7)
    mine = D.DeviceTokenLoader(FIX / "val_head.bin", T, bs, shuffle=shuffle, drop_last=drop_last, seed=7)
    for _ in range(2):  # two epochs: each draws a fresh permutation
        n = 0
        for rb, (x, y) in zip(ref, mine):
            assert tuple(x.shape) == rb["input"].shape and x.dtype == gpu.DType.Int64
            np.testing.assert_array_equal(_i64(gpu, x), rb["input"])
            np.testing.assert_array_equal(_i64(gpu, y), rb["target"])
            n += 1
        assert n == len(mine)


def test_token_windows_large_and_device_starts(gpu):
    rng = np.random.default_rng(0)
    toks = rng.integers(0, 50257, (1 << 20) + 3)
    ld = D.DeviceTokenLoader(toks, 256, 4096)
    starts = rng.integers(0, toks.size - 256, 4096)
    x, y = ld.batch(starts)
    want_x = toks[starts[:, None] + np.arange(256)]
    np.testing.assert_array_equal(_i64(gpu, x), want_x)
    np.testing.assert_array_equal(_i64(gpu, y), toks[starts[:, None] + np.arange(256) + 1])
    # starts already on the device
    ds = gpu.from_numpy(starts.astype(np.int64)).to(gpu.Device.CUDA)
    x2, _ = gpu._core._token_windows(ld.tokens, ds, 256)
    np.testing.assert_array_equal(_i64(gpu, x2), want_x)


def test_token_window_errors(gpu):
    toks = np.arange(50, dtype=np.int64)
    ld = D.DeviceTokenLoader(toks, 8, 2)
    with pytest.raises(IndexError):
        ld.batch([0, 42])  # 42 + 8 + 1 > 50: checked on the host
    with pytest.raises(IndexError):
        ld.batch([-1])
    x, y = ld.batch([41, 0])  # the last valid start
    np.testing.assert_array_equal(_i64(gpu, y)[0], np.arange(42, 50))
    # device-side starts: zeros, then IndexError at the next synchronisation
    bad = gpu.from_numpy(np.array([3, 45], np.int64)).to(gpu.Device.CUDA)
    x, _ = gpu._core._token_windows(ld.tokens, bad, 8)
    with pytest.raises(IndexError):
        _i64(gpu, x)
    x, _ = gpu._core._token_windows(ld.tokens, gpu.from_numpy(np.array([3], np.int64)).to(gpu.Device.CUDA), 8)
    np.testing.assert_array_equal(_i64(gpu, x)[0], np.arange(3, 11))  # the flag was cleared
    with pytest.raises(ValueError):
        gpu._core._token_windows(ld.tokens, gpu.from_numpy(np.array([0], np.int64)), 0)


def test_checkpoint_roundtrip_on_device(gpu, tmp_path):
    cfg = {"vocab_size": 65, "max_seq_len": 64, "n_layer": 2, "n_head": 4, "d_model": 128, "dropout": 0.0}
    a = lmutil.gpt_from_config(cfg, rng=np.random.default_rng(1))
    a.to(gpu.Device.CUDA)
    ids = D.read_tokens(FIX / "val_head.bin")[:4 * 64].reshape(4, 64)
    tid = gpu.from_numpy(np.ascontiguousarray(ids)).to(gpu.Device.CUDA)
    la = host(gpu, a(tid))
    ck.save_checkpoint(a, cfg, tmp_path / "ckpt_final")
    arrays, cfg2 = ck.read_checkpoint(tmp_path / "ckpt_final")
    assert cfg2["attn_bias"] is False and len(arrays) == 25
    b = lmutil.gpt_from_config(cfg2, rng=np.random.default_rng(2))
    b.to(gpu.Device.CUDA)
    ck.load_parameters(b, arrays, gpu.Device.CUDA)
    assert all(p.tensor.requires_grad for p in b.parameters())
    np.testing.assert_array_equal(host(gpu, b(tid)), la)


def test_shipped_checkpoint_runs_and_matches_oracle(gpu):
    arrays, cfg = ck.read_checkpoint(FIX / "ckpt_final")
    model = lmutil.gpt_from_config(cfg)
    model.to(gpu.Device.CUDA)
    ck.load_parameters(model, arrays, gpu.Device.CUDA)
    ids = np.ascontiguousarray(D.read_tokens(FIX / "val_head.bin")[:3 * 32].reshape(3, 32))
    logits = host(gpu, model(gpu.from_numpy(ids).to(gpu.Device.CUDA)))
    want = lmutil.oracle_forward(arrays, cfg, ids)
    assert_close(logits, want, 1e-4, "shipped checkpoint logits")
    # the shipped weights are barely trained (layernorm gains ~1, biases ~5e-3),
    # so only the loss itself is compared
    tgt = np.ascontiguousarray(D.read_tokens(FIX / "val_head.bin")[1:3 * 32 + 1])
    loss = host(gpu, gpu.cross_entropy(dev(gpu, logits.reshape(-1, 65)), gpu.from_numpy(tgt).to(gpu.Device.CUDA)))
    import oracle as O
    assert abs(float(loss) - float(O.cross_entropy(want.reshape(-1, 65), tgt))) < 1e-4
