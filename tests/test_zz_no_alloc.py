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
