"""On-disk formats of the reference's Shakespeare pipeline, host side: the
token file (raw little-endian int64), meta.json, the train/val split rule,
the window dataset and loader, and the checkpoint layout (.npz p0..pN + .json),
including the stale checkpoint the reference ships.  Fixtures under
tests/golden/shakespeare/ come from the reference's data directory
(tests/golden/make_data_fixtures.py)."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from aargrad import checkpoint as ck
from aargrad import data as D

FIX = Path(__file__).resolve().parent / "golden" / "shakespeare"


def test_token_file_and_vocab_encode_the_text():
    tok = D.CharTokenizer.load(FIX / "meta.json")
    assert tok.vocab_size == 65
    ids = D.read_tokens(FIX / "val_head.bin")
    assert ids.dtype == np.dtype("<i8") and ids.size == 8192
    text = (FIX / "val_head.txt").read_text()
    np.testing.assert_array_equal(tok.encode(text), ids)
    assert tok.decode(ids) == text
    # vocab is the sorted character set (data.py:13-15)
    assert tok.vocab == sorted(tok.vocab)


def test_split_rule_and_sizes():
    # prepare.py:40-47: val = last int(0.1 * len) ids, 8 bytes each
    f = json.loads((FIX / "facts.json").read_text())
    assert f["val_bin_bytes"] == 8 * f["val_tokens"]
    assert f["val_tokens"] == max(1, int(f["input_chars"] * 0.1)) == f["val_split_chars"]


def test_token_file_roundtrip(tmp_path):
    ids = np.random.default_rng(0).integers(0, 65, 1000)
    D.write_tokens(ids, tmp_path / "t.bin")
    assert (tmp_path / "t.bin").stat().st_size == 8000
    np.testing.assert_array_equal(np.fromfile(tmp_path / "t.bin", dtype="<i8"), ids)
    np.testing.assert_array_equal(D.read_tokens(tmp_path / "t.bin"), ids)


def test_meta_json_layout(tmp_path):
    tok = D.CharTokenizer.from_text("hello world")
    tok.save(tmp_path / "meta.json")
    assert json.loads((tmp_path / "meta.json").read_text()) == {"vocab": [" ", "d", "e", "h", "l", "o", "r", "w"],
                                                                 "vocab_size": 8}
    assert D.CharTokenizer.load(tmp_path / "meta.json").vocab == tok.vocab


def test_tokenizer_encode_decode_rules():
    # ids are positions in vocab (meta.json); unknown characters and ids raise
    # KeyError, as the reference's dict lookups do (data.py:7-33)
    tok = D.CharTokenizer(["b", "a", "\u00e9", "\n", "z"])
    np.testing.assert_array_equal(tok.encode("ab\u00e9\nz"), [1, 0, 2, 3, 4])
    assert tok.encode("").dtype == np.int64 and tok.encode("").shape == (0,)
    assert tok.decode([4, 3, 2, 1, 0]) == "z\n\u00e9ab"
    assert tok.decode(np.array([[0, 1]])) == "ba"
    assert tok.stoi["z"] == 4 and tok.itos[2] == "\u00e9" and tok.vocab_size == 5
    for bad in ("abc", "\u2603", "a\U0001F600"):
        with pytest.raises(KeyError):
            tok.encode(bad)
    for bad in ([5], [-1]):
        with pytest.raises(KeyError):
            tok.decode(bad)
    # the shipped vocabulary: every character of the validation text round-trips
    text = (FIX / "val_head.txt").read_text()
    ship = D.CharTokenizer.load(FIX / "meta.json")
    assert ship.decode(ship.encode(text)) == text
    np.testing.assert_array_equal(ship.encode(text), [ship.stoi[c] for c in text])


def test_dataset_indexing_and_collate():
    ids = np.arange(20, dtype=np.int64)
    ds = D.TokenWindowDataset(ids, 4)
    assert len(ds) == 16
    np.testing.assert_array_equal(ds[-1]["input"], ids[15:19])
    np.testing.assert_array_equal(ds[-1]["target"], ids[16:20])
    for bad in (16, -17):
        with pytest.raises(IndexError):
            ds[bad]
    assert [s["input"][0] for s in ds] == list(range(16))  # iteration stops at the end
    batch = [ds[i] for i in (3, 0, 7)]
    got = D.default_collate(batch)
    assert list(got) == ["input", "target"]
    for k in got:
        np.testing.assert_array_equal(got[k], np.stack([b[k] for b in batch]))
        assert got[k].dtype == np.int64 and got[k].shape == (3, 4)


def test_window_dataset_and_loader():
    ids = np.arange(100, dtype=np.int64) * 3
    ds = D.TokenWindowDataset(ids, 8)
    assert len(ds) == 92
    s = ds[5]
    np.testing.assert_array_equal(s["input"], ids[5:13])
    np.testing.assert_array_equal(s["target"], ids[6:14])
    ld = D.DataLoader(ds, 10, shuffle=True, seed=3)
    e1, e2 = list(ld), list(ld)
    assert len(e1) == 9 and all(b["input"].shape == (10, 8) for b in e1)
    starts = np.concatenate([b["input"][:, 0] // 3 for b in e1])
    assert len(set(starts.tolist())) == 90  # distinct windows, drop_last
    np.testing.assert_array_equal(np.concatenate([b["target"] for b in e1]),
                                  np.concatenate([b["input"] for b in e1]) + 3)
    assert not all(np.array_equal(a["input"], b["input"]) for a, b in zip(e1, e2))  # fresh order per epoch
    again = list(D.DataLoader(ds, 10, shuffle=True, seed=3))
    assert all(np.array_equal(a["input"], b["input"]) for a, b in zip(e1, again))
    tail = list(D.DataLoader(ds, 10, drop_last=False))
    assert len(tail) == 10 and tail[-1]["input"].shape == (2, 8)


def test_read_shipped_stale_checkpoint():
    arrays, cfg = ck.read_checkpoint(FIX / "ckpt_final")
    assert len(arrays) == 29
    assert cfg["max_seq_len"] == cfg["block_size"] == 32 and cfg["attn_bias"] is True
    D_, V = cfg["d_model"], cfg["vocab_size"]
    assert arrays[0].shape == (V, D_) and arrays[1].shape == (32, D_)
    assert arrays[4].shape == (3 * D_, D_) and arrays[5].shape == (3 * D_,)
    assert arrays[-1].shape == (V, D_) and all(a.dtype == np.float32 for a in arrays)


def _cpu_model(shapes, seed=0):
    import aargrad as ag
    from aargrad import nn

    class M(nn.Module):
        def __init__(self):
            super().__init__()
            rng = np.random.default_rng(seed)
            for i, s in enumerate(shapes):
                setattr(self, f"w{i}", nn.Parameter(ag.from_numpy(rng.standard_normal(s).astype(np.float32))))
    return M()


def test_checkpoint_layout_roundtrip(tmp_path):
    shapes = [(7, 3), (3,), (2, 2, 2)]
    m = _cpu_model(shapes)
    cfg = {"vocab_size": 7, "max_seq_len": 3, "n_layer": 0, "n_head": 1, "d_model": 3, "dropout": 0.0}
    ck.save_checkpoint(m, cfg, tmp_path / "ckpt_9")
    with np.load(tmp_path / "ckpt_9.npz") as z:
        assert sorted(z.files) == ["p0", "p1", "p2"]
        for i, p in enumerate(m.parameters()):
            import aargrad as ag
            np.testing.assert_array_equal(z[f"p{i}"], ag.to_numpy(p.tensor))
    assert (tmp_path / "ckpt_9.json").read_text() == json.dumps(cfg, indent=2)
    arrays, cfg2 = ck.read_checkpoint(tmp_path / "ckpt_9")
    assert cfg2["max_seq_len"] == 3 and len(arrays) == 3
    with pytest.raises(ValueError, match="param count mismatch"):
        ck.load_parameters(_cpu_model(shapes[:2]), arrays, None)
