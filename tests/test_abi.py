"""C-ABI checks that need no GPU: the library loads, exports every entry point
include/tsk/tsk.h declares, and rejects bad operands on the host before any
launch (the error conventions of include/tsk/tsk.h)."""
import ctypes
import os
import re

import pytest

from __graft_entry__ import ROOT, ensure_built, load_tsk

HEADER = os.path.join(ROOT, "include", "tsk", "tsk.h")


@pytest.fixture(scope="module")
def tsk():
    ensure_built()
    m = load_tsk()
    m.load()
    return m


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(tsk_[a-z0-9_]+)\s*\(", src)))


def test_exports_every_declared_symbol(tsk):
    names = declared_functions()
    assert len(names) >= 20
    lib = tsk.load()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_status_strings(tsk):
    lib = tsk.load()
    assert b"gfx950" in lib.tsk_version()
    assert lib.tsk_status_string(-3) == b"shape mismatch"
    assert lib.tsk_q8_0_split_nbytes(1024, 3072) == 1024 * 3072 + 2 * 3072 * 32
    assert lib.tsk_q8_0_split_nbytes(1000, 3) == 0


def fake(tsk, ttype, shape, elt):
    """descriptor with a non-null, aligned fake device address (never dereferenced)."""
    d = tsk.TskTensor()
    d.type = ttype
    ne = list(shape)[::-1] + [1] * (4 - len(shape))
    nb = [elt]
    for k in range(1, 4):
        nb.append(nb[-1] * ne[k - 1])
    for k in range(4):
        d.ne[k], d.nb[k] = ne[k], nb[k]
    d.data = 0x100000
    return d


def call_mm(tsk, a, b, dst, bias=None):
    lib = tsk.load()
    return lib.tsk_mul_mat(ctypes.byref(a), ctypes.byref(b), ctypes.byref(bias) if bias else None,
                           ctypes.byref(dst), None)


def test_mul_mat_validation(tsk):
    T = tsk
    a = fake(T, T.BF16, (3072, 1024), 2)
    b = fake(T, T.F32, (388, 1024), 4)
    dst = fake(T, T.F32, (388, 3072), 4)
    # valid operands reach the init check (no device work without tsk_init)
    assert call_mm(T, a, b, dst) == -7
    bad_b = fake(T, T.F32, (388, 1000), 4)
    assert call_mm(T, a, bad_b, dst) == -3                       # K mismatch
    bad_dst = fake(T, T.F32, (388, 3000), 4)
    assert call_mm(T, a, b, bad_dst) == -3                       # M mismatch
    assert call_mm(T, fake(T, T.F32, (3072, 1024), 4), b, dst) == -6   # F32 weights unsupported
    q = T.TskTensor()
    q.type = T.Q8_0
    q.ne[:] = [1000, 64, 1, 1]
    q.nb[:] = [34, 34 * 32, 34 * 32 * 64, 34 * 32 * 64]
    q.data = 0x100000
    assert call_mm(T, q, fake(T, T.F32, (5, 1000), 4), fake(T, T.F32, (5, 64), 4)) == -3   # K % 32
    nul = fake(T, T.F32, (388, 1024), 4)
    nul.data = None
    assert call_mm(T, a, nul, dst) == -1
    assert b"NULL" in T.load().tsk_last_error()
    mis = fake(T, T.F32, (388, 1024), 4)
    mis.data = 0x100004
    assert call_mm(T, a, mis, dst) == -5                         # misaligned
    strided = fake(T, T.F32, (388, 1024), 4)
    strided.nb[0] = 8
    assert call_mm(T, a, strided, dst) == -4                     # non-contiguous rows
    bias = fake(T, T.F32, (3072,), 4)
    assert call_mm(T, a, b, dst, bias) == -7
    assert call_mm(T, a, b, dst, fake(T, T.F32, (3071,), 4)) == -3


def test_flash_attn_validation(tsk):
    T = tsk
    lib = T.load()
    q = fake(T, T.F32, (1, 16, 420, 64), 4)
    k = fake(T, T.F16, (1, 16, 420, 64), 2)
    v = fake(T, T.F16, (1, 16, 420, 64), 2)
    dst = fake(T, T.F32, (1, 420, 16, 64), 4)
    fa = lambda q_, k_, v_, m_, d_, scale=0.125: lib.tsk_flash_attn_ext(
        ctypes.byref(q_), ctypes.byref(k_), ctypes.byref(v_), ctypes.byref(m_) if m_ else None,
        scale, 0.0, 0.0, 10, ctypes.byref(d_), None)
    assert fa(q, k, v, None, dst) == -7
    assert fa(fake(T, T.F32, (1, 16, 420, 128), 4), k, v, None, dst) == -6   # head dim 128
    assert fa(q, k, fake(T, T.BF16, (1, 16, 420, 64), 2), None, dst) == -2  # k/v types differ
    assert fa(q, k, v, None, fake(T, T.F32, (1, 16, 420, 64), 4)) == -3     # unpermuted dst
    assert fa(q, fake(T, T.F16, (1, 5, 420, 64), 2), fake(T, T.F16, (1, 5, 420, 64), 2), None, dst) == -3
    mask = fake(T, T.F16, (1, 1, 420, 420), 2)
    assert fa(q, k, v, mask, dst) == -7
    assert fa(q, k, v, fake(T, T.F16, (1, 1, 100, 420), 2), dst) == -3     # mask rows < Nq
    assert fa(q, k, v, None, dst, scale=0.0) == -1


def test_small_op_validation(tsk):
    T = tsk
    lib = T.load()
    x = fake(T, T.F32, (2, 194, 16, 64), 4)
    w = fake(T, T.F32, (64,), 4)
    pos = fake(T, T.I32, (194,), 4)
    y = fake(T, T.F32, (2, 194, 16, 64), 4)
    assert lib.tsk_rms_norm_mul(ctypes.byref(x), ctypes.byref(w), 1e-6, ctypes.byref(y), None) == -7
    assert lib.tsk_rms_norm_mul(ctypes.byref(x), ctypes.byref(fake(T, T.F32, (63,), 4)), 1e-6,
                                ctypes.byref(y), None) == -3
    assert lib.tsk_rope_ext(ctypes.byref(x), ctypes.byref(pos), 64, 0, 1e4, 1.0, 0.0, 1.0,
                            ctypes.byref(y), None) == -7
    assert lib.tsk_rope_ext(ctypes.byref(x), ctypes.byref(pos), 64, 2, 1e4, 1.0, 0.0, 1.0,
                            ctypes.byref(y), None) == -6               # NEOX mode not on the path
    assert lib.tsk_rope_ext(ctypes.byref(x), ctypes.byref(fake(T, T.I32, (77,), 4)), 64, 0, 1e4, 1.0,
                            0.0, 1.0, ctypes.byref(y), None) == -3
    assert lib.tsk_qk_norm_rope(ctypes.byref(x), ctypes.byref(w), None, 1e-6, 64, 1e4, 1.0,
                                ctypes.byref(y), None) == -7
    assert lib.tsk_norm(ctypes.byref(x), 1e-5, ctypes.byref(fake(T, T.F32, (2, 194, 16, 32), 4)), None) == -3


def test_supports_op(tsk):
    T = tsk
    lib = T.load()
    P = ctypes.POINTER(T.TskTensor)

    def sup(op, srcs, dst):
        arr = (P * len(srcs))(*[ctypes.pointer(s) if s is not None else P() for s in srcs])
        return lib.tsk_supports_op(op, arr, len(srcs), ctypes.byref(dst))

    a = fake(T, T.BF16, (1024, 1024), 2)
    b = fake(T, T.F32, (154, 1024), 4)
    d = fake(T, T.F32, (154, 1024), 4)
    assert sup(T.OP_MUL_MAT, [a, b], d) == 1
    assert sup(T.OP_MUL_MAT, [fake(T, T.F32, (1024, 1024), 4), b], d) == 0
    q = fake(T, T.F32, (1, 16, 77, 64), 4)
    kv = fake(T, T.F16, (1, 16, 77, 64), 2)
    o = fake(T, T.F32, (1, 77, 16, 64), 4)
    assert sup(T.OP_FLASH_ATTN_EXT, [q, kv, kv], o) == 1
    assert sup(T.OP_FLASH_ATTN_EXT, [fake(T, T.F32, (1, 8, 77, 80), 4), kv, kv], o) == 0
