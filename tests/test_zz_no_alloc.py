"""The no-allocation attention entry point (ae_attention_varlen_noalloc, static device scratch)
against the allocating operator ae_attention_varlen, through the C ABI."""
import ctypes

import numpy as np
import pytest

import arctic_embed_amd as ae

pytestmark = pytest.mark.gpu


def _call(lib, qkv, cu, n, t, max_len, ctx):
    return lib.ae_attention_varlen_noalloc(ctypes.c_void_p(qkv), ctypes.c_void_p(cu), n, t, max_len,
                                           ctypes.c_void_p(ctx), None)


def test_noalloc_attention_matches_allocating_operator(torch_gpu):
    """Bit-identical to ae_attention_varlen on consecutive calls, the later ones smaller (the
    static plan keeps the last call's records: each call must rewrite what it reads), through the
    tiled kernels and the short-row kernels; sizes past the static scratch are refused."""
    torch = torch_gpu
    lib = ae.lib()
    rng = np.random.default_rng(7)
    for lens in ([130, 512, 7, 64, 1, 300, 33, 257], [100, 3, 70, 9], [40, 2, 17]):
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
        T = int(cu[-1])
        print("noalloc attention lens", lens, flush=True)
        qkv = torch.from_numpy(rng.normal(0, 1.0, (T, 1152)).astype(np.float32)).cuda()
        cu_d = torch.from_numpy(cu).cuda()
        ref = torch.full((T, 384), float("nan"), dtype=torch.float32, device="cuda")
        out = torch.full((T, 384), float("nan"), dtype=torch.float32, device="cuda")
        ae.attention_varlen(qkv.data_ptr(), cu_d.data_ptr(), len(lens), T, ref.data_ptr())
        torch.cuda.synchronize()
        assert _call(lib, qkv.data_ptr(), cu_d.data_ptr(), len(lens), T, max(lens), out.data_ptr()) == ae.AE_OK
        torch.cuda.synchronize()
        r, o = ref.cpu().numpy(), out.cpu().numpy()
        assert np.all(np.isfinite(r))
        assert np.array_equal(r.view(np.uint32), o.view(np.uint32)), lens
    # past the static scratch (524288 plan records, two lists): refused before any launch
    assert _call(lib, 1, 1, 60000, 1 << 20, 512, 1) == ae.AE_ERR_CAPACITY
    assert "static scratch" in ae.lib().ae_last_error().decode()
    assert _call(lib, 1, 1, 2, 100, 513, 1) == ae.AE_ERR_INVALID_ARG
