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


@pytest.fixture
def uninit(tsk):
    """The validation checks below pass descriptors whose device address is
    fake and expect TSK_ERR_NOT_INIT for the nodes that pass validation: once
    tsk_init has run in this process (an earlier GPU test), such a node would
    be launched on the fake address, so these checks run only before it."""
    if tsk._initialised:
        pytest.skip("tsk_init already ran in this process: valid nodes with fake addresses would be launched")
    return tsk


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


def test_mul_mat_validation(uninit):
    T = uninit
    a = fake(T, T.BF16, (3072, 1024), 2)
    b = fake(T, T.F32, (388, 1024), 4)
    dst = fake(T, T.F32, (388, 3072), 4)
    # valid operands reach the init check (no device work without tsk_init)
    assert call_mm(T, a, b, dst) == -7
    bad_b = fake(T, T.F32, (388, 1000), 4)
    assert call_mm(T, a, bad_b, dst) == -3                       # K mismatch
    bad_dst = fake(T, T.F32, (388, 3000), 4)
    assert call_mm(T, a, b, bad_dst) == -3                       # M mismatch
    assert call_mm(T, fake(T, T.F32, (3072, 1024), 4), b, dst) == -7   # F32 weights: all-fp32 GEMM
    assert call_mm(T, fake(T, T.F16, (3072, 1024), 2), b, dst) == -6   # F16 weights unsupported
    assert call_mm(T, fake(T, T.F32, (3072, 1024), 4), fake(T, T.BF16, (388, 1024), 2), dst) == -2
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


def test_flash_attn_validation(uninit):
    T = uninit
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


def test_small_op_validation(uninit):
    T = uninit
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
    assert sup(T.OP_MUL_MAT, [fake(T, T.F32, (1024, 1024), 4), b], d) == 1
    assert sup(T.OP_MUL_MAT, [fake(T, T.F16, (1024, 1024), 2), b], d) == 0
    q = fake(T, T.F32, (1, 16, 77, 64), 4)
    kv = fake(T, T.F16, (1, 16, 77, 64), 2)
    o = fake(T, T.F32, (1, 77, 16, 64), 4)
    assert sup(T.OP_FLASH_ATTN_EXT, [q, kv, kv], o) == 1
    assert sup(T.OP_FLASH_ATTN_EXT, [fake(T, T.F32, (1, 8, 77, 80), 4), kv, kv], o) == 0


def kernel_desc(T, ttype, oc, ic, kw, es, kw_major=False):
    """ggml conv kernel ne = [KW, IC, OC]; ggml layout or the kw-major one"""
    d = fake(T, ttype, (oc, ic, kw), es)
    if kw_major:
        d.nb[0], d.nb[1], d.nb[2] = ic * es, es, kw * ic * es
    return d


def test_conv_validation(uninit):
    T = uninit
    lib = T.load()
    w = kernel_desc(T, T.BF16, 2816, 1024, 3, 2)
    x = fake(T, T.F32, (2, 646, 1024), 4)          # ne [IC, IW, B]
    y = fake(T, T.F32, (2, 646, 2816), 4)
    conv = lambda w_, x_, y_, s0=1, p0=1, d0=1, b_=None: lib.tsk_conv1d(
        ctypes.byref(w_), ctypes.byref(b_) if b_ else None, ctypes.byref(x_), s0, p0, d0, ctypes.byref(y_), None)
    assert conv(w, x, y) == -7
    assert conv(kernel_desc(T, T.BF16, 2816, 1024, 3, 2, True), x, y) == -7
    assert conv(kernel_desc(T, T.F32, 2816, 1024, 3, 4), x, y) == -7
    assert conv(kernel_desc(T, T.Q8_0, 2816, 1024, 3, 1), x, y) == -2        # 3-D kernels are BF16 / F32
    assert conv(w, x, fake(T, T.F32, (2, 645, 2816), 4)) == -3              # OW mismatch
    assert conv(w, x, fake(T, T.F32, (2, 323, 2816), 4), s0=2) == -7        # stride 2: OW = 323
    assert conv(w, x, y, p0=-1) == -1
    assert conv(kernel_desc(T, T.BF16, 64, 20, 3, 2), fake(T, T.F32, (1, 30, 20), 4),
                fake(T, T.F32, (1, 30, 64), 4)) == -3                        # IC % 8
    assert conv(kernel_desc(T, T.F32, 64, 16, 3, 4), fake(T, T.BF16, (1, 30, 16), 2),
                fake(T, T.F32, (1, 30, 64), 4)) == -2                        # F32 kernel, BF16 x
    assert conv(w, x, y, b_=fake(T, T.F32, (2816,), 4)) == -7
    assert conv(w, x, y, b_=fake(T, T.F32, (2815,), 4)) == -3
    # im2col node: x ne [IW, IC, N] any strides, dst [IC*KW, OW, N]
    xi = fake(T, T.F32, (1, 1024, 646), 4)
    ci = fake(T, T.F32, (1, 646, 3072), 4)
    im = lambda x_, d_, s0=1, p0=1, d0=1: lib.tsk_im2col_1d(ctypes.byref(w), ctypes.byref(x_), s0, p0, d0,
                                                            ctypes.byref(d_), None)
    assert im(xi, ci) == -7
    assert im(xi, fake(T, T.F16, (1, 646, 3072), 2)) == -7
    assert im(xi, fake(T, T.F32, (1, 646, 3000), 4)) == -3
    assert im(fake(T, T.F16, (1, 1024, 646), 2), ci) == -2
    # SwiGLU MLPs
    w2 = kernel_desc(T, T.BF16, 1024, 2816, 3, 2)
    out = fake(T, T.F32, (2, 646, 1024), 4)
    cm = lambda a, b_, c, x_, d_: lib.tsk_conv_mlp_swiglu(ctypes.byref(a), ctypes.byref(b_), ctypes.byref(c),
                                                          ctypes.byref(x_), ctypes.byref(d_), None)
    assert cm(w, w, w2, x, out) == -7
    assert cm(w, w, kernel_desc(T, T.F32, 1024, 2816, 3, 4), x, out) == -2    # mixed kernel types
    assert cm(w, w, kernel_desc(T, T.BF16, 1024, 2000, 3, 2), x, out) == -3   # w2 IC != HID
    l1 = fake(T, T.BF16, (2816, 1024), 2)
    l2 = fake(T, T.BF16, (1024, 2816), 2)
    xt = fake(T, T.F32, (154, 1024), 4)
    ml = lambda a, b_, c, x_, d_: lib.tsk_mlp_swiglu(ctypes.byref(a), ctypes.byref(b_), ctypes.byref(c),
                                                     ctypes.byref(x_), ctypes.byref(d_), None)
    assert ml(l1, l1, l2, xt, fake(T, T.F32, (154, 1024), 4)) == -7
    assert ml(l1, l1, l2, xt, fake(T, T.F32, (154, 1000), 4)) == -3
    a = fake(T, T.F32, (646, 2816), 4)
    assert lib.tsk_swiglu(ctypes.byref(a), ctypes.byref(a), ctypes.byref(a), None) == -7
    assert lib.tsk_swiglu(ctypes.byref(a), ctypes.byref(fake(T, T.F32, (646, 2815), 4)), ctypes.byref(a),
                          None) == -3
    # kw-major pack: dst strides must be the kw-major ones
    pk = kernel_desc(T, T.BF16, 2816, 1024, 3, 2, True)
    assert lib.tsk_conv1d_pack_weight(ctypes.byref(w), ctypes.byref(pk), None) == -7
    assert lib.tsk_conv1d_pack_weight(ctypes.byref(w), ctypes.byref(w), None) == -4


def test_workspace_size(tsk):
    """tsk_workspace_size: the scratch each node takes from its stream's
    workspace, computed on the host from the descriptors (no GPU, no init)."""
    T = tsk
    lib = T.load()
    P = ctypes.POINTER(T.TskTensor)

    def ws(op, srcs, dst):
        arr = (P * len(srcs))(*[ctypes.pointer(s) if s is not None else P() for s in srcs])
        n = ctypes.c_size_t(12345)
        rc = lib.tsk_workspace_size(op, arr, len(srcs), ctypes.byref(dst), ctypes.byref(n))
        return rc, n.value

    a = fake(T, T.BF16, (3072, 1024), 2)
    assert ws(T.OP_MUL_MAT, [a, fake(T, T.F32, (388, 1024), 4)], fake(T, T.F32, (388, 3072), 4)) == (0, 388 * 1024 * 2)
    assert ws(T.OP_MUL_MAT, [a, fake(T, T.BF16, (388, 1024), 2)], fake(T, T.F32, (388, 3072), 4)) == (0, 0)
    assert ws(T.OP_MUL_MAT, [a, fake(T, T.F32, (388, 1000), 4)], fake(T, T.F32, (388, 3072), 4))[0] == -3
    q = T.TskTensor()
    q.type = T.Q8_0
    q.ne[:] = [1024, 64, 1, 1]
    q.nb[:] = [34, 34 * 32, 34 * 32 * 64, 34 * 32 * 64]
    q.data = 0x100000
    # repacked weights (aligned to 256) + activation planes (int8 rows, then f32 block scales)
    wbytes = (1024 * 64 + 2 * 64 * 32 + 255) // 256 * 256
    act = (5 * 1024 + 4 * 5 * 32 + 255) // 256 * 256
    assert ws(T.OP_MUL_MAT, [q, fake(T, T.F32, (5, 1024), 4)], fake(T, T.F32, (5, 64), 4)) == (0, wbytes + act)
    qf = fake(T, T.F32, (1, 16, 420, 64), 4)
    kv = fake(T, T.F16, (1, 16, 420, 64), 2)
    o = fake(T, T.F32, (1, 420, 16, 64), 4)
    assert ws(T.OP_FLASH_ATTN_EXT, [qf, kv, kv], o) == (0, 0)          # F16 V read as rows: no scratch
    kvb = fake(T, T.BF16, (1, 16, 420, 64), 2)
    assert ws(T.OP_FLASH_ATTN_EXT, [qf, kvb, kvb], o) == (0, 2 * 16 * 64 * 448)     # bf16 V: V^T, fp16, 64-key padded
    assert ws(T.OP_FLASH_ATTN_EXT, [qf, kv, kv, fake(T, T.F16, (1, 1, 420, 420), 2)], o) == (0, 0)   # masked: none
    w = kernel_desc(T, T.BF16, 2816, 1024, 3, 2)                    # ggml layout: packed per call
    x = fake(T, T.F32, (2, 646, 1024), 4)
    y = fake(T, T.F32, (2, 646, 2816), 4)
    assert ws(T.OP_CONV1D, [w, x], y) == (0, 3 * 1024 * 2816 * 2 + 2 * 646 * 1024 * 2)
    assert ws(T.OP_CONV1D, [kernel_desc(T, T.BF16, 2816, 1024, 3, 2, True), x], y) == (0, 2 * 646 * 1024 * 2)
    xt = fake(T, T.F32, (2, 200, 2048), 4)
    qd = T.TskTensor()
    qd.type = T.Q8_0
    qd.ne[:] = [2048, 200, 2, 1]
    qd.nb[:] = [34, 64 * 34, 64 * 34 * 200, 64 * 34 * 400]
    qd.data = 0x100000
    # int8 planes [400][2048] and f32 scales [400][64]
    assert ws(T.OP_RMS_NORM_Q8_0, [xt, fake(T, T.F32, (2048,), 4)], qd) == (0, 400 * 2048 + 400 * 64 * 4)
    assert ws(T.OP_RMS_NORM_MUL, [xt], xt) == (0, 0)
    assert ws(99, [xt], xt)[0] == -6
