"""tsk_mul_mat_noalloc: tsk_mul_mat with its scratch in the library's fixed
per-GPU array (no allocation). Compared bit for bit with tsk_mul_mat on two
calls in a row, the second with a smaller input, for every kind of scratch
the node takes (f32 activations rounded to bf16 rows; Q8_0 blocks repacked
plus the quantized activation planes; repacked Q8_0 planes with activation
planes only), and a node needing more than the array is refused before any
launch."""
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


def q8_blocks(rng, M, K):
    qs = rng.integers(-127, 128, size=(M, K // 32, 32), dtype=np.int8)
    d = (np.abs(rng.standard_normal((M, K // 32, 1))) * 2e-4 + 1e-5).astype(np.float16).view(np.uint8)
    return np.ascontiguousarray(np.concatenate([d, qs.view(np.uint8)], axis=2))


def weights(tsk, rng, kind, K, M):
    if kind == "bf16":
        return tsk.bf16_to_device(bf16_bits(rng.standard_normal((M, K)) * 0.02)), None
    blocks = tsk.to_device(q8_blocks(rng, M, K))
    if kind == "q8_0":
        return blocks, tsk.Q8_0
    return tsk.q8_0_repack(blocks), tsk.Q8_0_SPLIT


@pytest.mark.parametrize("kind", ["bf16", "q8_0", "q8_0_split"])
def test_noalloc_matches_mul_mat_two_calls(tsk, kind):
    rng = np.random.default_rng({"bf16": 1, "q8_0": 2, "q8_0_split": 3}[kind])
    K, M = 1024, 3072
    w, at = weights(tsk, rng, kind, K, M)
    bias = tsk.to_device((rng.standard_normal(M) * 0.1).astype(np.float32))
    for N in (1446, 388):                 # second call smaller: stale scratch must not leak in
        x = tsk.to_device(rng.standard_normal((N, K)).astype(np.float32))
        y_ref = tsk.mul_mat(w, x, bias=bias, a_type=at)
        y = tsk.mul_mat_noalloc(w, x, bias=bias, a_type=at)
        tsk.synchronize()
        a, b = y.numpy(), y_ref.numpy()
        assert np.isfinite(a).all()
        assert np.array_equal(a, b), f"{kind} N={N}: max |diff| {np.abs(a - b).max()}"


def test_noalloc_refuses_oversized_node(tsk):
    """a node whose scratch exceeds the fixed array is rejected with
    TSK_ERR_NOMEM before anything is launched"""
    rng = np.random.default_rng(4)
    K, M = 4096, 256
    w = tsk.bf16_to_device(bf16_bits(rng.standard_normal((M, K)) * 0.02))
    N = (32 << 20) // (2 * K) + 16        # bf16 rows of N x K exceed 32 MiB
    x = tsk.empty((N, K))
    y = tsk.empty((N, M))
    with pytest.raises(tsk.TskError) as ei:
        tsk.mul_mat_noalloc(w, x, out=y)
    assert ei.value.status == -9 and "limit" in str(ei.value)
    # bf16 activations need no scratch at all: any size runs
    xb = tsk.bf16_to_device(bf16_bits(rng.standard_normal((300, K))))
    yb = tsk.mul_mat_noalloc(w, xb)
    yr = tsk.mul_mat(w, xb)
    tsk.synchronize()
    assert np.array_equal(yb.numpy(), yr.numpy())


def test_noalloc_under_graph_capture(tsk):
    """tsk_mul_mat_noalloc is for callers under HIP graph capture: a BF16 and
    a Q8_0 node (both staging their activations in the fixed array) captured
    on one stream in Global mode (a hipMalloc or other call not allowed under
    capture would fail it), replayed three times with eager work and
    synchronisations between the replays; every replay gives the bits of
    tsk_mul_mat"""
    rng = np.random.default_rng(7)
    K, M, N = 1024, 3072, 388
    wb, _ = weights(tsk, rng, "bf16", K, M)
    wq, atq = weights(tsk, rng, "q8_0", K, M)
    bias = tsk.to_device((rng.standard_normal(M) * 0.1).astype(np.float32))
    x1 = tsk.to_device(rng.standard_normal((N, K)).astype(np.float32))
    x2 = tsk.to_device(rng.standard_normal((N, K)).astype(np.float32))
    r1 = tsk.mul_mat(wb, x1, bias=bias).numpy()
    r2 = tsk.mul_mat(wq, x2, a_type=atq).numpy()
    s = tsk.Stream()
    y1, y2 = tsk.empty((N, M)), tsk.empty((N, M))
    # first launches of these kernels outside the capture
    tsk.mul_mat_noalloc(wb, x1, bias=bias, out=y1, stream=s)
    tsk.mul_mat_noalloc(wq, x2, a_type=atq, out=y2, stream=s)
    s.synchronize()

    def work():
        tsk.mul_mat_noalloc(wb, x1, bias=bias, out=y1, stream=s)
        tsk.mul_mat_noalloc(wq, x2, a_type=atq, out=y2, stream=s)
    g = tsk.Graph(s, work)
    try:
        for rep in range(3):
            nan = np.full((N, M), np.nan, np.float32)
            for y in (y1, y2):                       # eager work between replays
                tsk._hipcheck(tsk.hip().hipMemcpy(y.data_ptr(), nan.ctypes.data, nan.nbytes, 1), "reset")
            tsk.mul_mat(wq, x1, a_type=atq)          # other scratch traffic on the null stream
            tsk.synchronize()
            g.launch()
            s.synchronize()
            assert np.array_equal(y1.numpy(), r1), f"replay {rep}: bf16 node"
            assert np.array_equal(y2.numpy(), r2), f"replay {rep}: Q8_0 node"
    finally:
        g.destroy()
        s.destroy()
