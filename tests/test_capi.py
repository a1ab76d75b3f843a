"""The C-ABI library loads and exports every entry point include/hynomas.h declares (no GPU needed)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hynomas.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hn_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared()
    for expected in ("hn_quantize_act", "hn_block_gemm", "hn_adaln", "hn_adaln_quant", "hn_gated_residual",
                     "hn_qk_norm_rope", "hn_pixelumm_qk", "hn_version", "hn_last_error"):
        assert expected in names


def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (the library binds to torch's HIP runtime)
    from hy_nomas import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libhynomas_hip.so not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == set(declared())


def test_argument_validation_without_a_gpu():
    """Bad shapes are rejected on the host before any launch, with a message."""
    import torch  # noqa: F401
    from hy_nomas import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libhynomas_hip.so not built")
    l = _lib.lib()
    assert l.hn_version() >= 100
    rc = l.hn_quantize_act(None, 0, 100, 4, 100, 128, 0, 0, None, 100, None, 1, None)   # K % 128 != 0
    assert rc == 1 and b"multiple of 128" in l.hn_last_error()
    rc = l.hn_block_gemm(None, 256, None, 2, None, 256, None, 2, 1, None, 0, 4, 8, 256, 64, 0, 0, None, 0, 8, None,
                         0, None)   # group 64
    assert rc == 1 and b"group" in l.hn_last_error()
    rc = l.hn_adaln_quant(None, None, None, 0, 1, 4, 200, 1e-6, 0, 0, 128, None, None, None)   # D % 128 != 0
    assert rc == 1 and b"multiple of 128" in l.hn_last_error()
    rc = l.hn_qk_norm_rope(None, 96, None, None, None, 1, 1, 1, 96, 1e-6, None, None)   # head dim 96
    assert rc == 1
    rc = l.hn_block_gemm(None, 256, None, 2, None, 256, None, 2, 1, None, 0, 4, 8, 256, 128, 0, 7, None, 0, 8, None,
                         0, None)   # bad epilogue
    assert rc == 1
    rc = l.hn_block_gemm(None, 256, None, 2, None, 256, None, 2, 64, None, 0, 4, 8, 256, 128, 1, 0, None, 0, 8, None,
                         0, None)   # weight-scale rows of 64 channels
    assert rc == 1 and b"sw_rows" in l.hn_last_error()
    rc = l.hn_block_gemm(None, 256, None, 1, None, 256, None, 1, 128, None, 0, 4, 8, 256, 256, 1, 0, None, 0, 8, None,
                         0, None)   # block weight scales need group 128
    assert rc == 1 and b"sw_rows" in l.hn_last_error()
    rc = l.hn_block_gemm(None, 256, None, 2, None, 256, None, 2, 128, None, 0, 4, 384, 256, 128, 1, 4, None, 0, 192,
                         None, 1, None)   # swiglu_quant over 384 rows: not whole gate/up pairs of 256
    assert rc == 1 and b"swiglu_quant" in l.hn_last_error()
    rc = l.hn_block_gemm(None, 256, None, 2, None, 256, None, 2, 128, None, 0, 4, 512, 256, 128, 1, 4, None, 0, 256,
                         None, 1, None)   # swiglu_quant scales [M, N/256] missing
    assert rc == 1 and b"swiglu_quant" in l.hn_last_error()
    rc = l.hn_qkv_heads(None, 256, None, 2, None, 256, None, 2, 1, None, 0, 1, 64, 200, 256, 128, 0, None, None,
                        None, None, 1e-6, None, 64, 0, None)   # hidden 200: not whole 128-channel heads
    assert rc == 1 and b"hidden" in l.hn_last_error()
    rc = l.hn_qkv_heads(None, 256, None, 2, None, 256, None, 2, 1, None, 0, 1, 64, 256, 256, 128, 0, None, None,
                        None, None, 1e-6, None, 70, 10, None)  # tokens [10, 74) past L_total 70
    assert rc == 1 and b"L_total" in l.hn_last_error()
    rc = l.hn_qkv_heads_vt(None, 256, None, 2, None, 256, None, 2, 1, None, 0, 1, 48, 256, 256, 128, 0, None, None,
                           None, None, 1e-6, None, 64, 0, 16, 128 * 64 * 2, 128 * 64, 64, None)   # L = 48
    assert rc == 1 and b"multiple of 32" in l.hn_last_error()
    rc = l.hn_qkv_heads_vt(None, 256, None, 2, None, 256, None, 2, 1, None, 0, 1, 64, 256, 256, 128, 0, None, None,
                           None, None, 1e-6, None, 64, 0, 16, 128 * 32 * 2, 128 * 32, 32, None)   # rows of 32 keys < 64
    assert rc == 1 and b"V^T strides" in l.hn_last_error()
    rc = l.hn_gated_residual_frames(None, None, None, None, 0, 1, 2, 3, 100, None, None)   # D % 8 != 0
    assert rc == 1 and b"multiple of 8" in l.hn_last_error()
    rc = l.hn_block_gemm(None, 131072, None, 1, None, 131072, None, 1, 1, None, 0, 4, 8, 131072, 131072, 0, 0, None,
                         0, 8, None, 0, None)   # int8 whole-K over 2^17: the int32 sum could overflow
    assert rc == 1 and b"overflow" in l.hn_last_error()
    rc = l.hn_block_gemm(None, 131072, None, 1024, None, 131072, None, 1024, 1, None, 0, 4, 8, 131072, 128, 0, 3,
                         None, 0, 8, None, 0, None)   # ACC32 always sums the whole K in int32
    assert rc == 1 and b"overflow" in l.hn_last_error()


def test_attention_argument_validation_without_a_gpu():
    """hn_attention rejects, on the host: a head dim other than 128, V^T rows shorter than the key tiles, strides
    past the 32-bit tile offsets, and a non-positive scale (non-null, 16-byte aligned dummy pointers that are
    never dereferenced, since every case fails before a launch)."""
    import torch  # noqa: F401
    from hy_nomas import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libhynomas_hip.so not built")
    l = _lib.lib()
    p = 4096  # a 16-byte aligned address the checks never read

    def call(D=128, svd=128, skj=128, scale=0.088, Lk=100):
        return l.hn_attention(p, 0, 0, 128, p, 0, 0, skj, p, 0, 0, svd, p, 0, 0, 128, 1, 1, 10, Lk, D, scale, None)

    assert call(D=96) == 1 and b"head dim" in l.hn_last_error()
    assert call(svd=64) == 1 and b"V^T rows" in l.hn_last_error()
    assert call(skj=1 << 24) == 1 and b"out of range" in l.hn_last_error()
    assert call(scale=0.0) == 1 and b"scale" in l.hn_last_error()
    assert call(Lk=0) == 1 and b"bad shape" in l.hn_last_error()


def test_noalloc_rejects_problems_beyond_the_scratch():
    """hn_block_linear_noalloc refuses, before any HIP call, a problem whose codes and scales exceed the scratch
    array the header declares.  The size is read from the header, so a larger array keeps the case out of
    range.  Runs only where no GPU is visible: the pointers passed are placeholders."""
    import torch
    from hy_nomas import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libhynomas_hip.so not built")
    if torch.cuda.is_available():
        pytest.skip("placeholder pointers: host-only check")
    text = open(HEADER).read()
    scratch = eval(re.search(r"#define HN_NOALLOC_SCRATCH_BYTES\s+\(([^)]*)\)", text).group(1).replace("LL", ""))
    l = _lib.lib()
    k = 3072
    m = scratch // k + 1
    assert l.hn_block_linear_workspace_bytes(m, k, 128) > scratch
    assert l.hn_block_linear_workspace_bytes(m, k, k) > scratch
    for group in (128, k):
        rc = l.hn_block_linear_noalloc(1 << 20, 0, k, m, k, group, 0, 0, 1 << 20, k, 1 << 20, k // 128, 1, None, 0,
                                       256, 1 << 20, 0, 256, None)
        assert rc == 1 and b"scratch" in l.hn_last_error()
    # and a problem just inside the array is within the limit
    fits = scratch // (k + 4 * (k // 128)) - 1
    assert 0 < l.hn_block_linear_workspace_bytes(fits, k, 128) <= scratch
