"""Writes the data-format fixtures under tests/golden/shakespeare/ from the
reference's shipped Shakespeare data (python/shakespeare/data/):

  meta.json             the vocabulary file, copied
  ckpt_final.npz/.json  the shipped checkpoint, copied (the stale one: its
                        config says block_size and it carries attention biases)
  val_head.bin          the first 8192 tokens of val.bin (raw little-endian int64)
  val_head.txt          the text those tokens encode: the first 8192 characters
                        of the validation split of input.txt (the last
                        int(0.1 * len) characters, prepare.py:41-43)
  facts.json            sizes the reference's files have (val.bin bytes and
                        token count, input.txt characters)

Run in the container that holds the reference tree:
    python tests/golden/make_data_fixtures.py
"""
from __future__ import annotations

import json
import shutil
from pathlib import Path

import numpy as np

SRC = Path("/root/reference/python/shakespeare/data")
OUT = Path(__file__).resolve().parent / "shakespeare"
HEAD = 8192


def main() -> None:
    if not SRC.is_dir():
        raise SystemExit(f"{SRC} not found (needs the reference tree)")
    OUT.mkdir(exist_ok=True)
    for name in ("meta.json", "ckpt_final.npz", "ckpt_final.json"):
        shutil.copyfile(SRC / name, OUT / name)
    val = np.fromfile(SRC / "val.bin", dtype="<i8")
    val[:HEAD].tofile(OUT / "val_head.bin")
    text = (SRC / "input.txt").read_text()
    n_val = max(1, int(len(text) * 0.1))
    (OUT / "val_head.txt").write_text(text[-n_val:][:HEAD])
    facts = {"val_bin_bytes": (SRC / "val.bin").stat().st_size, "val_tokens": int(val.size),
             "input_chars": len(text), "val_split_chars": n_val}
    (OUT / "facts.json").write_text(json.dumps(facts, indent=2) + "\n")


if __name__ == "__main__":
    main()
