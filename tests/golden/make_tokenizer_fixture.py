"""Writes tests/golden/tokenizer_vectors.json and tests/golden/vocab.txt.

Source: the reference's own test data files (read as data, never executed):
  tests/data/reference_test_vectors.json  -> 12 records: kind, raw_text, ids
  tests/data/long_texts.txt + tests/data/long_reference_vectors.json -> 7 records
  model/vocab.txt (the WordPiece vocabulary)
The records' embedding_fp32 fields are dropped: they pin the forward pass only
with the real model.ae8, which is not available offline.

Usage (in a container where the reference tree is mounted):
  python tests/golden/make_tokenizer_fixture.py /root/reference
"""
import json
import os
import shutil
import sys


def main(ref):
    here = os.path.dirname(os.path.abspath(__file__))
    recs = json.load(open(os.path.join(ref, "tests/data/reference_test_vectors.json"), encoding="utf-8"))
    short = [{"kind": r["kind"], "raw_text": r["raw_text"], "ids": r["ids"]} for r in recs]
    lines = [l for l in open(os.path.join(ref, "tests/data/long_texts.txt"), encoding="utf-8").read().split("\n")
             if l.strip()]
    longs = json.load(open(os.path.join(ref, "tests/data/long_reference_vectors.json"), encoding="utf-8"))
    assert len(lines) == len(longs)
    long_recs = [{"name": r["name"], "text": t, "ids": r["ids"]} for r, t in zip(longs, lines)]
    with open(os.path.join(here, "tokenizer_vectors.json"), "w", encoding="utf-8") as f:
        json.dump({"short": short, "long": long_recs}, f, ensure_ascii=False, indent=0)
    shutil.copyfile(os.path.join(ref, "model/vocab.txt"), os.path.join(here, "vocab.txt"))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
