"""ctypes binding of liboracle.so -- the CPU parity oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product library.  See oracle.h.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
if not os.path.exists(LIB_PATH):
    raise ImportError("liboracle.so is not built (make -C %s)" % _HERE)
_lib = ctypes.CDLL(LIB_PATH)

H, I, LAYERS, VOCAB, MAX_POS = 384, 1536, 12, 30522, 512
OR_OK, OR_ERR_IO, OR_ERR_INVALID_DATA, OR_ERR_EOF, OR_ERR_ARG = 0, -1, -2, -3, -4

_vp = ctypes.c_void_p
_fp = ctypes.POINTER(ctypes.c_float)


class _Linear(ctypes.Structure):
    _fields_ = [("n_out", ctypes.c_uint64), ("k_in", ctypes.c_uint64), ("w_len", ctypes.c_uint64),
                ("s_len", ctypes.c_uint64), ("b_len", ctypes.c_uint64), ("is_len", ctypes.c_uint64),
                ("w_q", ctypes.POINTER(ctypes.c_int8)), ("w_scale", _fp), ("bias", _fp), ("inv_smooth", _fp),
                ("xpack", ctypes.POINTER(ctypes.c_int8)), ("xcomp", ctypes.POINTER(ctypes.c_int32))]


class _Layer(ctypes.Structure):
    _fields_ = [("qkv", _Linear), ("has_split", ctypes.c_int), ("q_only", _Linear), ("kv_only", _Linear),
                ("attn_out", _Linear), ("ln1_w", _fp), ("ln1_b", _fp), ("ln1_w_len", ctypes.c_uint64),
                ("ln1_b_len", ctypes.c_uint64), ("ffn_inter", _Linear), ("ffn_out", _Linear), ("ln2_w", _fp),
                ("ln2_b", _fp), ("ln2_w_len", ctypes.c_uint64), ("ln2_b_len", ctypes.c_uint64)]


class _Model(ctypes.Structure):
    _fields_ = [("word_q", ctypes.POINTER(ctypes.c_int8)), ("word_q_len", ctypes.c_uint64),
                ("word_s", _fp), ("word_s_len", ctypes.c_uint64),
                ("pos_q", ctypes.POINTER(ctypes.c_int8)), ("pos_q_len", ctypes.c_uint64),
                ("pos_s", _fp), ("pos_s_len", ctypes.c_uint64),
                ("type_q", ctypes.POINTER(ctypes.c_int8)), ("type_q_len", ctypes.c_uint64),
                ("type_s", _fp), ("type_s_len", ctypes.c_uint64),
                ("emb_ln_w", _fp), ("emb_ln_w_len", ctypes.c_uint64),
                ("emb_ln_b", _fp), ("emb_ln_b_len", ctypes.c_uint64),
                ("layers", _Layer * LAYERS), ("type0", ctypes.c_float * H)]


_MP = ctypes.POINTER(_Model)
_sigs = {
    "or_load_ae8": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_MP)]),
    "or_free": (None, [_MP]),
    "or_size_bytes": (ctypes.c_size_t, [_MP]),
    "or_gemm": (None, [ctypes.c_int, _vp, _vp, ctypes.POINTER(_Linear), _vp, _vp]),
    "or_gemm_acc": (None, [ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, _vp, _vp]),
    "or_ln_quant_row": (ctypes.c_float, [_vp, _vp, _vp, _vp, _vp, ctypes.c_int, ctypes.c_float]),
    "or_ln_row": (None, [_vp, _vp, _vp, ctypes.c_int, ctypes.c_float]),
    "or_smooth_quant_row": (ctypes.c_float, [_vp, _vp, _vp, ctypes.c_int]),
    "or_gelu": (ctypes.c_float, [ctypes.c_float]),
    "or_gelu_map": (None, [_vp, _vp, ctypes.c_size_t]),
    "or_gelu_quant_row": (ctypes.c_float, [_vp, _vp, _vp, ctypes.c_int]),
    "or_dot32": (ctypes.c_float, [_vp, _vp]),
    "or_scores": (None, [_vp, _vp, ctypes.c_float, _vp, ctypes.c_int]),
    "or_softmax": (None, [_vp, ctypes.c_int]),
    "or_wsum": (None, [_vp, _vp, ctypes.c_int, _vp]),
    "or_emb_row": (None, [_vp, ctypes.c_float, _vp, ctypes.c_float, _vp, _vp, ctypes.c_int]),
    "or_l2": (None, [_vp, ctypes.c_int]),
    "or_attention_head": (None, [_vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp,
                                 ctypes.c_int]),
    "or_attention_sme": (None, [_vp, ctypes.c_int, _vp, ctypes.c_int, _vp]),
    "or_exp2_q": (ctypes.c_int32, [ctypes.c_float, ctypes.c_float, ctypes.c_float]),
    "or_forward_cls": (ctypes.c_int, [_MP, _vp, ctypes.c_size_t, _vp]),
    "or_forward_cls_unpruned": (ctypes.c_int, [_MP, _vp, ctypes.c_size_t, _vp]),
    "or_forward_ragged_cls": (ctypes.c_int, [_MP, _vp, _vp, ctypes.c_int, _vp]),
    "or_embed_batch_tokens": (ctypes.c_int, [_MP, _vp, _vp, ctypes.c_size_t, ctypes.c_int, _vp]),
    "or_x86_backend": (ctypes.c_int, []),
    "or_x86_gemm": (ctypes.c_int, [ctypes.c_int, _vp, _vp, ctypes.POINTER(_Linear), _vp, _vp, ctypes.c_int]),
    "or_x86_prepare": (ctypes.c_int, [_MP]),
    "or_x86_embed_batch_tokens": (ctypes.c_int, [_MP, _vp, _vp, ctypes.c_size_t, ctypes.c_int, _vp]),
    "or_run_prefix": (ctypes.c_int, [_MP, _vp, _vp, ctypes.c_int, ctypes.c_int, _vp, _vp, _vp]),
    "or_run_prefix_sme": (ctypes.c_int, [_MP, _vp, _vp, ctypes.c_int, ctypes.c_int, _vp, _vp, _vp]),
    "or_embed_tokens_sme": (ctypes.c_int, [_MP, _vp, _vp, ctypes.c_int, _vp]),
    "or_forward_cls_perturbed": (ctypes.c_int, [_MP, _vp, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                _vp]),
}
for _n, (_r, _a) in _sigs.items():
    _f = getattr(_lib, _n)
    _f.restype = _r
    _f.argtypes = _a


def _f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def _arr(ptr, n, dtype):
    if n == 0:
        return np.zeros(0, dtype=dtype)
    ctype = np.ctypeslib.as_ctypes_type(dtype)
    return np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctype)), shape=(n,)).copy()


class LinearView:
    """Copy of one QuantizedLinearRaw's vectors."""

    def __init__(self, lin):
        self.n_out, self.k_in = int(lin.n_out), int(lin.k_in)
        self.w_q = _arr(lin.w_q, lin.w_len, np.int8).reshape(self.n_out, self.k_in) if lin.w_len else \
            np.zeros((0, self.k_in), np.int8)
        self.w_scale = _arr(lin.w_scale, lin.s_len, np.float32)
        self.bias = _arr(lin.bias, lin.b_len, np.float32)
        self.inv_smooth = _arr(lin.inv_smooth, lin.is_len, np.float32)


def x86_gemm(a_q, a_scale, w_q, w_scale, bias, res=None, variant=1):
    """The x86 baseline's GEMM (variant 1: AVX2 maddubs, 2: AVX-VNNI) on the same operands as gemm()."""
    a_q = np.ascontiguousarray(a_q, dtype=np.int8)
    w_q = np.ascontiguousarray(w_q, dtype=np.int8)
    m, k = a_q.shape
    n = w_q.shape[0]
    ws, b = _f32(w_scale), _f32(bias)
    inv = np.ones(k, np.float32)
    lin = _Linear(n, k, n * k, n, n, k, w_q.ctypes.data_as(ctypes.POINTER(ctypes.c_int8)),
                  ws.ctypes.data_as(_fp), b.ctypes.data_as(_fp), inv.ctypes.data_as(_fp))
    sc = _f32(a_scale)
    out = np.zeros((m, n), np.float32)
    r = None if res is None else _f32(res)
    rc = _lib.or_x86_gemm(m, a_q.ctypes.data, sc.ctypes.data, ctypes.byref(lin),
                          None if r is None else r.ctypes.data, out.ctypes.data, int(variant))
    # the packed copies belong to this temporary linear
    libc_free = ctypes.CDLL(None).free
    libc_free.argtypes = [ctypes.c_void_p]
    libc_free(ctypes.cast(lin.xpack, ctypes.c_void_p))
    libc_free(ctypes.cast(lin.xcomp, ctypes.c_void_p))
    if rc:
        raise ValueError("or_x86_gemm: %d" % rc)
    return out


def x86_backend():
    """The reference's x86 backend on this host: 'avx_vnni', 'avx2' or None (src/gemm.rs:100-125)."""
    return {2: "avx_vnni", 1: "avx2"}.get(int(_lib.or_x86_backend()))


def _pack(seqs):
    lens = [len(s) for s in seqs]
    offsets = np.zeros(len(seqs) + 1, dtype=np.uint32)
    offsets[1:] = np.cumsum(lens)
    ids = np.concatenate([np.asarray(s, dtype=np.uint16) for s in seqs]) if seqs else np.zeros(1, np.uint16)
    return np.ascontiguousarray(ids, dtype=np.uint16), offsets


class OracleModel:
    def __init__(self, path):
        self._m = _MP()
        rc = _lib.or_load_ae8(str(path).encode(), ctypes.byref(self._m))
        self.status = rc
        if rc != OR_OK:
            self._m = None
            raise OSError(rc, "or_load_ae8 failed with %d" % rc)

    def close(self):
        if self._m:
            _lib.or_free(self._m)
            self._m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def raw(self):
        return self._m.contents

    def size_bytes(self):
        return int(_lib.or_size_bytes(self._m))

    def layer(self, i):
        return self._m.contents.layers[i]

    def linear(self, layer, name):
        return LinearView(getattr(self._m.contents.layers[layer], name))

    def linear_ptr(self, layer, name):
        return ctypes.pointer(getattr(self._m.contents.layers[layer], name))

    def vec(self, layer, name):
        L = self._m.contents.layers[layer]
        return _arr(getattr(L, name), getattr(L, name + "_len"), np.float32)

    def forward_cls(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint16)
        out = np.zeros(H, dtype=np.float32)
        rc = _lib.or_forward_cls(self._m, ids.ctypes.data, ids.size, out.ctypes.data)
        if rc:
            raise ValueError("or_forward_cls: %d" % rc)
        return out

    def forward_cls_perturbed(self, ids, layer, row, col):
        """forward_cls with act_q[row][col] one int8 step off at the input of encoder layer `layer`."""
        ids = np.ascontiguousarray(ids, dtype=np.uint16)
        out = np.zeros(H, dtype=np.float32)
        rc = _lib.or_forward_cls_perturbed(self._m, ids.ctypes.data, ids.size, int(layer), int(row), int(col),
                                           out.ctypes.data)
        if rc:
            raise ValueError("or_forward_cls_perturbed: %d" % rc)
        return out

    def forward_cls_unpruned(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint16)
        out = np.zeros(H, dtype=np.float32)
        rc = _lib.or_forward_cls_unpruned(self._m, ids.ctypes.data, ids.size, out.ctypes.data)
        if rc:
            raise ValueError("or_forward_cls_unpruned: %d" % rc)
        return out

    def forward_ragged_cls(self, seqs):
        ids, offs = _pack(seqs)
        out = np.zeros((len(seqs), H), dtype=np.float32)
        rc = _lib.or_forward_ragged_cls(self._m, ids.ctypes.data, offs.ctypes.data, len(seqs), out.ctypes.data)
        if rc:
            raise ValueError("or_forward_ragged_cls: %d" % rc)
        return out

    def embed_batch_tokens(self, seqs, num_threads=1):
        ids, offs = _pack(seqs)
        out = np.zeros((len(seqs), H), dtype=np.float32)
        rc = _lib.or_embed_batch_tokens(self._m, ids.ctypes.data, offs.ctypes.data, len(seqs), int(num_threads),
                                        out.ctypes.data)
        if rc:
            raise ValueError("or_embed_batch_tokens: %d" % rc)
        return out

    def x86_embed_batch_tokens(self, seqs, num_threads=1):
        """embed_batch on the restated x86 backend of the reference (AVX-VNNI or AVX2, chosen as the
        reference chooses): the CPU baseline.  Not bit-identical to the scalar oracle."""
        if not getattr(self, "_x86_ready", False):
            rc = _lib.or_x86_prepare(self._m)
            if rc:
                raise ValueError("or_x86_prepare: %d (no AVX2+FMA?)" % rc)
            self._x86_ready = True
        ids, offs = _pack(seqs)
        out = np.zeros((len(seqs), H), dtype=np.float32)
        rc = _lib.or_x86_embed_batch_tokens(self._m, ids.ctypes.data, offs.ctypes.data, len(seqs), int(num_threads),
                                            out.ctypes.data)
        if rc:
            raise ValueError("or_x86_embed_batch_tokens: %d" % rc)
        return out

    def embed_tokens_sme(self, seqs):
        """forward_cls of every sequence with the ArmSme backend's quantized attention (>= 16 tokens)."""
        ids, offs = _pack(seqs)
        out = np.zeros((len(seqs), H), dtype=np.float32)
        rc = _lib.or_embed_tokens_sme(self._m, ids.ctypes.data, offs.ctypes.data, len(seqs), out.ctypes.data)
        if rc:
            raise ValueError("or_embed_tokens_sme: %d" % rc)
        return out

    def run_prefix_sme(self, seqs, upto_layer):
        """run_prefix with the ArmSme backend's quantized attention in layers 0-10."""
        return self.run_prefix(seqs, upto_layer, sme=True)

    def run_prefix(self, seqs, upto_layer, sme=False):
        ids, offs = _pack(seqs)
        T = int(offs[-1])
        hidden = np.zeros((T, H), np.float32)
        act_q = np.zeros((T, H), np.int8)
        scale = np.zeros(T, np.float32)
        fn = _lib.or_run_prefix_sme if sme else _lib.or_run_prefix
        rc = fn(self._m, ids.ctypes.data, offs.ctypes.data, len(seqs), int(upto_layer),
                hidden.ctypes.data, act_q.ctypes.data, scale.ctypes.data)
        if rc:
            raise ValueError("or_run_prefix: %d" % rc)
        return hidden, act_q, scale


def load_status(path):
    m = _MP()
    rc = _lib.or_load_ae8(str(path).encode(), ctypes.byref(m))
    if rc == OR_OK:
        _lib.or_free(m)
    return rc


# ---- kernel-level functions (numpy in, numpy out) ----

def gemm(a_q, a_scale, w_q, w_scale, bias, res=None):
    """gemm_scalar_fused (src/gemm.rs:2000-2029)."""
    a_q = np.ascontiguousarray(a_q, dtype=np.int8)
    w_q = np.ascontiguousarray(w_q, dtype=np.int8)
    m, k = a_q.shape
    n = w_q.shape[0]
    ws, b = _f32(w_scale), _f32(bias)
    inv = np.ones(k, np.float32)
    lin = _Linear(n, k, n * k, n, n, k, w_q.ctypes.data_as(ctypes.POINTER(ctypes.c_int8)),
                  ws.ctypes.data_as(_fp), b.ctypes.data_as(_fp), inv.ctypes.data_as(_fp))
    sc = _f32(a_scale)
    out = np.zeros((m, n), np.float32)
    r = None if res is None else _f32(res)
    _lib.or_gemm(m, a_q.ctypes.data, sc.ctypes.data, ctypes.byref(lin), None if r is None else r.ctypes.data,
                 out.ctypes.data)
    return out


def gemm_acc(a_q, w_q):
    a_q = np.ascontiguousarray(a_q, dtype=np.int8)
    w_q = np.ascontiguousarray(w_q, dtype=np.int8)
    m, k = a_q.shape
    n = w_q.shape[0]
    acc = np.zeros((m, n), np.int32)
    _lib.or_gemm_acc(m, n, k, a_q.ctypes.data, w_q.ctypes.data, acc.ctypes.data)
    return acc


def ln_quant_rows(x, gamma, beta, inv_smooth, eps=1e-12):
    """layernorm_smooth_quantize_row_scalar over rows; returns (y, q, scale)."""
    x = _f32(x).copy()
    m, n = x.shape
    q = np.zeros((m, n), np.int8)
    sc = np.zeros(m, np.float32)
    g, b, s = _f32(gamma), _f32(beta), _f32(inv_smooth)
    for r in range(m):
        sc[r] = _lib.or_ln_quant_row(x[r].ctypes.data, g.ctypes.data, b.ctypes.data, s.ctypes.data,
                                     q[r].ctypes.data, n, eps)
    return x, q, sc


def ln_rows(x, gamma, beta, eps=1e-12):
    x = _f32(x).copy()
    g, b = _f32(gamma), _f32(beta)
    for r in range(x.shape[0]):
        _lib.or_ln_row(x[r].ctypes.data, g.ctypes.data, b.ctypes.data, x.shape[1], eps)
    return x


def smooth_quant_rows(x, inv_smooth):
    x = _f32(x)
    m, n = x.shape
    q = np.zeros((m, n), np.int8)
    sc = np.zeros(m, np.float32)
    s = _f32(inv_smooth)
    for r in range(m):
        sc[r] = _lib.or_smooth_quant_row(x[r].ctypes.data, s.ctypes.data, q[r].ctypes.data, n)
    return q, sc


def gelu(x):
    """scalar_gelu (src/simd_math.rs:15-23) elementwise."""
    x = _f32(x)
    y = np.empty_like(x)
    _lib.or_gelu_map(x.ctypes.data, y.ctypes.data, x.size)
    return y


def gelu_quant_rows(x, inv_smooth):
    """gelu_smooth_quantize_row scalar; returns (g, q, scale)."""
    x = _f32(x).copy()
    m, n = x.shape
    q = np.zeros((m, n), np.int8)
    sc = np.zeros(m, np.float32)
    s = _f32(inv_smooth)
    for r in range(m):
        sc[r] = _lib.or_gelu_quant_row(x[r].ctypes.data, s.ctypes.data, q[r].ctypes.data, n)
    return x, q, sc


def softmax(s):
    s = _f32(s).copy()
    _lib.or_softmax(s.ctypes.data, s.size)
    return s


def dot32(a, b):
    a, b = _f32(a), _f32(b)
    return float(_lib.or_dot32(a.ctypes.data, b.ctypes.data))


def wsum(p, v):
    p, v = _f32(p), _f32(v)
    out = np.zeros(32, np.float32)
    _lib.or_wsum(p.ctypes.data, v.ctypes.data, p.size, out.ctypes.data)
    return out


def emb_row(w_row, w_s, p_row, p_s, t_row):
    w_row = np.ascontiguousarray(w_row, np.int8)
    p_row = np.ascontiguousarray(p_row, np.int8)
    t_row = _f32(t_row)
    out = np.zeros(w_row.size, np.float32)
    _lib.or_emb_row(w_row.ctypes.data, float(w_s), p_row.ctypes.data, float(p_s), t_row.ctypes.data,
                    out.ctypes.data, w_row.size)
    return out


def l2(v):
    v = _f32(v).copy()
    _lib.or_l2(v.ctypes.data, v.size)
    return v


def attention(qkv, cu):
    """Segment-bounded attention of one layer over qkv [T,1152] (src/model.rs:663-694)."""
    qkv = _f32(qkv)
    T = qkv.shape[0]
    ctx = np.zeros((T, H), np.float32)
    for b in range(len(cu) - 1):
        s0, L = int(cu[b]), int(cu[b + 1] - cu[b])
        for h in range(12):
            _lib.or_attention_head(qkv[s0:].ctypes.data, L, 3 * H, h * 32, H + h * 32, 2 * H + h * 32,
                                   ctx[s0:, h * 32:].ctypes.data, H)
    return ctx


def attention_sme(qkv, cu):
    """The reference's quantized (ArmSme) attention over a packed batch
    (src/model.rs:607-621, src/simd_math.rs:1933-2192)."""
    qkv = _f32(qkv)
    cu = np.ascontiguousarray(cu, np.int32)
    T = qkv.shape[0]
    ctx = np.zeros((T, H), np.float32)
    _lib.or_attention_sme(qkv.ctypes.data, T, cu.ctypes.data, len(cu) - 1, ctx.ctypes.data)
    return ctx


def exp2_q(x, scale=16383.0, x_min=-16.0):
    """exp2_q_neon for one lane (src/simd_math.rs:2353-2370)."""
    return int(_lib.or_exp2_q(float(x), float(scale), float(x_min)))
