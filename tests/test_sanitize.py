"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer.

tests/sanitize/Makefile builds the product's .ae8 loader (csrc/ae8.cpp), its
tokenizer (csrc/tokenizer.cpp) and the CPU oracle (oracle/oracle.c, x86.c) with
g++/gcc -fsanitize=address,undefined (no GPU code), into one driver.  Each test
runs one mode of the driver: any sanitizer report aborts it (-fno-sanitize-recover),
and its outputs must equal what the unsanitized libraries return for the same
inputs, bit for bit."""
import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import arctic_embed_amd as ae
import oracle as orc
from conftest import GOLDEN, ROOT

SAN_DIR = os.path.join(ROOT, "tests", "sanitize")
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1:strict_string_checks=1",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if shutil.which("g++") is None or shutil.which("make") is None:
        pytest.skip("host compiler not available")
    out = tmp_path_factory.mktemp("sanitize_build")
    r = subprocess.run(["make", "-s", "-C", SAN_DIR, "OUT=%s" % out, "-j4"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return str(out / "driver")


def _run(args, timeout=300):
    r = subprocess.run(args, capture_output=True, text=True, env=ENV, timeout=timeout)
    assert r.returncode == 0, "driver failed (%d):\n%s\n%s" % (r.returncode, r.stdout, r.stderr[-4000:])
    assert "runtime error" not in r.stderr and "Sanitizer" not in r.stderr, r.stderr[-4000:]
    return r.stdout


def test_loader_under_sanitizers(driver, tmp_path):
    """Synthetic pack write + load through both loaders, the bad-magic and missing-file
    errors, 258 truncation points (each must read as UnexpectedEof) and trailing bytes."""
    out = _run([driver, "loader", str(tmp_path)])
    assert out.startswith("loader: ")


EDGE_TEXTS = [
    b"", b" ", b"\t\n\r", b"a", b"a" * 100, b"a" * 101, b"word " * 700,
    b"\xff\xfe\xfd", b"abc\xe4\xb8", b"\xc0\xaf", b"\xed\xa0\x80x", b"\xf4\x90\x80\x80",
    "café CAFÉ café Ångström".encode(), "中文字 あ".encode(),
    "\U0001F600\U0001F680 emoji".encode(), " 　  spaces".encode(),
    b"!!!???...,,,;;;" * 20, b"x\x00y", b"\x07\x1b[31m", "İstanbul ẞ".encode(),
    "ΑΒΓ АБВ".encode(), b"don't can't it's-a mid-word",
]


def test_tokenizer_under_sanitizers(driver, tmp_path):
    """The reference's own id vectors plus malformed UTF-8, overlong words, >512 tokens,
    CJK, combining marks and control characters, single-threaded and batched."""
    d = json.load(open(os.path.join(GOLDEN, "tokenizer_vectors.json"), encoding="utf-8"))
    fixture = [(e["kind"] == "query", e["raw_text"].encode("utf-8"), e["ids"]) for e in d["short"]]
    fixture += [(False, e["text"].encode("utf-8"), e["ids"]) for e in d["long"]]
    cases = fixture + [(q, t, None) for t in EDGE_TEXTS for q in (False, True)]
    rec = b"".join(struct.pack("<BI", int(q), len(t)) + t for q, t, _ in cases)
    (tmp_path / "in.bin").write_bytes(rec)
    _run([driver, "tokenize", os.path.join(GOLDEN, "vocab.txt"), str(tmp_path / "in.bin"),
          str(tmp_path / "out.bin")])
    raw = (tmp_path / "out.bin").read_bytes()
    n = struct.unpack_from("<I", raw)[0]
    assert n == len(cases)
    offs = np.frombuffer(raw, np.uint32, n + 1, 4)
    ids = np.frombuffer(raw, np.uint16, int(offs[-1]), 4 + 4 * (n + 1))
    tok = ae.Tokenizer(os.path.join(GOLDEN, "vocab.txt"))
    try:
        for i, (q, t, want) in enumerate(cases):
            got = ids[offs[i]:offs[i + 1]].tolist()
            assert 2 <= len(got) <= 512 and got[0] == 101 and got[-1] == 102, i
            if want is not None:
                assert got == want, i
            elif b"\x00" not in t:
                # the unsanitized product library, through its C ABI
                buf = np.zeros(512, np.uint16)
                cnt = ae.ctypes.c_size_t()
                ae._check(ae._lib.ae_tokenizer_encode(tok._h, t, int(q), buf.ctypes.data, buf.size,
                                                      ae.ctypes.byref(cnt)))
                assert got == buf[:cnt.value].tolist(), (i, t)
    finally:
        tok.close()


def _qkv_lcg(T):
    """The driver's seeded qkv rows: 64-bit LCG, top 24 bits, centred, / 2^22."""
    s = 0x9E3779B97F4A7C15
    out = np.empty(T * 1152, np.float32)
    m = (1 << 64) - 1
    for i in range(out.size):
        s = (s * 6364136223846793005 + 1442695040888963407) & m
        out[i] = np.float32((s >> 40) - (1 << 23)) * np.float32(1.0 / (1 << 22))
    return out.reshape(T, 1152)


def test_oracle_under_sanitizers(driver, tmp_path, model_dir, oracle_model):
    """Every oracle driver (forward_cls, ragged, embed_batch at 1 and 4 threads, the x86
    backend, the ArmSme-attention forward) and both attention kernels, sanitized,
    against the unsanitized oracle library: identical bits."""
    rng = np.random.default_rng(7)
    lens = [2, 15, 16, 33, 60]
    seqs = [np.concatenate([[101], rng.integers(1000, 30522, L - 2), [102]]).astype(np.uint16) for L in lens]
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    blob = struct.pack("<I", len(seqs)) + offs.tobytes() + np.concatenate(seqs).tobytes()
    (tmp_path / "in.bin").write_bytes(blob)
    _run([driver, "oracle", str(model_dir / "model.ae8"), str(tmp_path / "in.bin"), str(tmp_path / "out.bin")],
         timeout=600)
    got = np.fromfile(str(tmp_path / "out.bin"), np.float32)
    B, H = len(seqs), 384
    want = [oracle_model.forward_cls(seqs[0]).reshape(-1), oracle_model.forward_ragged_cls(seqs).reshape(-1),
            oracle_model.embed_batch_tokens(seqs, 1).reshape(-1), oracle_model.embed_batch_tokens(seqs, 4).reshape(-1)]
    m2 = orc.OracleModel(str(model_dir / "model.ae8"))  # x86 packing stays off the shared model
    try:
        want.append(m2.x86_embed_batch_tokens(seqs, 2).reshape(-1))
    finally:
        m2.close()
    want.append(oracle_model.embed_tokens_sme(seqs).reshape(-1))
    cu = np.array([0, 1, 19, 52], np.int32)
    qkv = _qkv_lcg(int(cu[-1]))
    want.append(orc.attention(qkv, cu).reshape(-1))
    want.append(orc.attention_sme(qkv, cu).reshape(-1))
    want = np.concatenate(want)
    assert got.size == want.size == H + 5 * B * H + 2 * int(cu[-1]) * H
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
