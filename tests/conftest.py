import os
import shutil
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "snowflake-arctic-embed-s-rust_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

MODEL_SEED = 0xAE85EED
# sha256 of the synthetic pack for MODEL_SEED (pins the generator byte-for-byte)
MODEL_SHA256 = "0a0b5339de942d973347242c123e6ed969005df5fe971bbae8ab4b044c37a989"
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X)")


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    import arctic_embed_amd as ae
    d = tmp_path_factory.mktemp("model")
    ae.write_synthetic_ae8(str(d / "model.ae8"), MODEL_SEED)
    shutil.copyfile(os.path.join(GOLDEN, "vocab.txt"), str(d / "vocab.txt"))
    return d


@pytest.fixture(scope="session")
def oracle_model(model_dir):
    import oracle as orc
    m = orc.OracleModel(str(model_dir / "model.ae8"))
    yield m
    m.close()


def c1_ids():
    """[CLS] + 126 ids U[1000,30522) + [SEP], seed 1."""
    rng = np.random.default_rng(1)
    return np.concatenate([[101], rng.integers(1000, 30522, 126), [102]]).astype(np.uint16)


def ragged_batch(n, lo, hi, seed):
    """n sequences, total length U{lo..hi} including [CLS]/[SEP], body ids U[1000,30522)."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, n)
    return [np.concatenate([[101], rng.integers(1000, 30522, int(L) - 2), [102]]).astype(np.uint16)
            for L in lens]


@pytest.fixture(scope="session")
def torch_gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch
