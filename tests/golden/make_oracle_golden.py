"""Writes tests/golden/oracle_golden.json: oracle outputs on the seeded synthetic
model (seed 0xAE85EED) that pin the oracle and the pack generator against
regressions.  Regenerate only after an intended change to either.

Usage: python tests/golden/make_oracle_golden.py
"""
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "snowflake-arctic-embed-s-rust_amd"), os.path.join(ROOT, "oracle"),
                os.path.join(ROOT, "tests")]
import arctic_embed_amd as ae  # noqa: E402
import oracle as orc  # noqa: E402
from conftest import MODEL_SEED, c1_ids, ragged_batch  # noqa: E402


def main():
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "model.ae8")
        ae.write_synthetic_ae8(path, MODEL_SEED)
        m = orc.OracleModel(path)
        c1 = m.forward_cls(c1_ids())
        seqs = ragged_batch(8, 16, 96, 3)
        rag = m.embed_batch_tokens(seqs, 4)
        out = {
            "model_seed": MODEL_SEED,
            "c1_embedding": [float(x) for x in c1],
            "ragged_seed3_n8_16_96": [[float(x) for x in row] for row in rag],
        }
        m.close()
    with open(os.path.join(HERE, "oracle_golden.json"), "w") as f:
        json.dump(out, f)


if __name__ == "__main__":
    main()
