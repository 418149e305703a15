"""Workspaces of the C ABI (include/tsk/tsk.h): every operator that needs
device scratch takes it from the workspace of its stream, so calls on two
streams from two host threads run concurrently without sharing scratch, and a
caller can bind its own buffer (sized by tsk_workspace_size) so that the
library allocates nothing. Checked bit for bit against serial runs."""
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tsk():
    from __graft_entry__ import ensure_built, load_tsk
    ensure_built()
    m = load_tsk()
    m.init(0)
    return m


def bf16_bits(a):
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def operands(tsk, seed):
    """a BF16 GEMM with f32 activations (scratch: the bf16 rows) and a fast-path
    flash attention with bf16 K / V (scratch: V transposed to fp16; F16 V is
    read as rows and takes none), two different sizes per seed"""
    rng = np.random.default_rng(seed)
    N = 300 + 50 * seed
    w = tsk.bf16_to_device(bf16_bits(rng.standard_normal((1024, 1024)) * 0.02))
    x = tsk.to_device(rng.standard_normal((N, 1024)).astype(np.float32))
    nq = 200 + 70 * seed
    q = tsk.to_device(rng.standard_normal((2, 16, nq, 64)).astype(np.float32))
    k = tsk.bf16_to_device(bf16_bits(rng.standard_normal((2, 16, nq, 64))))
    v = tsk.bf16_to_device(bf16_bits(rng.standard_normal((2, 16, nq, 64))))
    return w, x, q, k, v


def run_ops(tsk, ops, stream, reps):
    """the two operators `reps` times on `stream` into one pair of outputs
    allocated up front (no allocation or free while the stream runs)"""
    w, x, q, k, v = ops
    y = tsk.empty((x.shape[0], w.shape[0]))
    o = tsk.empty((q.shape[0], q.shape[2], q.shape[1], 64))
    for _ in range(reps):
        tsk.mul_mat(w, x, out=y, stream=stream)
        tsk.flash_attn_ext(q, k, v, scale=0.125, out=o, stream=stream)
    return y, o


def test_two_streams_two_threads_match_serial(tsk):
    ops = [operands(tsk, s) for s in (1, 2)]
    # serial reference on the null stream
    ref = []
    for op in ops:
        y, o = run_ops(tsk, op, None, 1)
        tsk.synchronize()
        ref.append((y.numpy(), o.numpy()))
    streams = [tsk.Stream(), tsk.Stream()]
    out = [None, None]
    errors = []

    def worker(i):
        try:
            y, o = run_ops(tsk, ops[i], streams[i], 20)
            streams[i].synchronize()
            out[i] = (y.numpy(), o.numpy())
        except Exception as e:      # reported on the main thread
            errors.append(e)

    th = [threading.Thread(target=worker, args=(i,)) for i in (0, 1)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errors, errors
    for i in (0, 1):
        assert np.array_equal(out[i][0], ref[i][0])
        assert np.array_equal(out[i][1], ref[i][1])
    for s in streams:
        s.destroy()


def test_bound_workspace_exact_size(tsk):
    """tsk_workspace_size reports what the node needs: bound at exactly that
    size the call succeeds with the same bits, 256 bytes short it is refused
    with TSK_ERR_NOMEM (the library does not fall back to allocating)."""
    w, x, q, k, v = operands(tsk, 3)
    y_ref = tsk.mul_mat(w, x)
    o_ref = tsk.flash_attn_ext(q, k, v, scale=0.125)
    tsk.synchronize()
    y_ref, o_ref = y_ref.numpy(), o_ref.numpy()
    y = tsk.empty((x.shape[0], 1024))
    o = tsk.empty((2, q.shape[2], 16, 64))
    n_mm = tsk.workspace_size(tsk.OP_MUL_MAT, [w, x], y)
    n_fa = tsk.workspace_size(tsk.OP_FLASH_ATTN_EXT, [q, k, v], o)
    assert n_mm == x.shape[0] * 1024 * 2                         # f32 rows rounded to bf16
    assert n_fa == 2 * 2 * 16 * 64 * ((q.shape[2] + 63) // 64 * 64)   # V^T, fp16
    s = tsk.Stream()
    buf = tsk.empty((max(n_mm, n_fa),), "u8")
    tsk.set_workspace(buf, stream=s)
    tsk.mul_mat(w, x, out=y, stream=s)
    tsk.flash_attn_ext(q, k, v, scale=0.125, out=o, stream=s)
    s.synchronize()
    assert np.array_equal(y.numpy(), y_ref) and np.array_equal(o.numpy(), o_ref)
    small = tsk.empty((n_mm - 256,), "u8")
    tsk.set_workspace(small, stream=s)
    with pytest.raises(tsk.TskError) as ei:
        tsk.mul_mat(w, x, out=y, stream=s)
    assert ei.value.status == -9
    tsk.set_workspace(None, stream=s)      # unbound: the library's own buffer again
    tsk.mul_mat(w, x, out=y, stream=s)
    s.synchronize()
    assert np.array_equal(y.numpy(), y_ref)
    s.destroy()
