"""mul_mat on gfx950 (BF16 and Q8_0 weights) through the C ABI vs the oracle.
BF16/Q8_0 GEMM output rel-L2 <= 1e-3; Q8_0 (de)quantization bit-exact."""
import numpy as np
import pytest

import refmath
from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env(orc):
    from __graft_entry__ import ensure_built, load_tsk
    ensure_built()
    tsk = load_tsk()
    tsk.init(0)
    return tsk, orc


SHAPES_BF16 = [(388, 1024, 3072), (388, 1024, 1024), (542, 1024, 4096), (388, 4096, 1024),
               (154, 2048, 1024), (194, 3072, 2816), (194, 8448, 1024), (2, 1024, 6144),
               (1, 64, 1024), (7, 40, 12), (1446, 1024, 3072), (1292, 1024, 6144)]


@pytest.mark.parametrize("N,K,M", SHAPES_BF16)
def test_bf16_gemm(env, N, K, M):
    tsk, orc = env
    rng = np.random.default_rng(N * 7 + M)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    wb = orc.f32_to_bf16_bits(w)
    x = rng.standard_normal((N, K)).astype(np.float32)
    bias = rng.standard_normal(M).astype(np.float32) if M % 4 == 0 else None
    y = tsk.mul_mat(tsk.bf16_to_device(wb), tsk.to_device(x),
                    bias=tsk.to_device(bias) if bias is not None else None)
    yref = orc.mul_mat(wb, x, bias=bias, a_type=orc.BF16)
    assert rel_l2(y.numpy(), yref) <= 1e-3


def test_bf16_gemm_bf16_activations_and_output(env):
    tsk, orc = env
    rng = np.random.default_rng(11)
    M, K, N = 3072, 1024, 388
    wb = orc.f32_to_bf16_bits((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    xb = orc.f32_to_bf16_bits(rng.standard_normal((N, K)).astype(np.float32))
    y = tsk.mul_mat(tsk.bf16_to_device(wb), tsk.bf16_to_device(xb), out_dtype="bf16")
    yref = orc.mul_mat(wb, orc.bf16_bits_to_f32(xb), a_type=orc.BF16)
    assert rel_l2(orc.bf16_bits_to_f32(y.numpy()), yref) <= 5e-3
    # exact closed form: products of bf16 values are exact in fp32
    yf = tsk.mul_mat(tsk.bf16_to_device(wb), tsk.bf16_to_device(xb)).numpy()
    exact = orc.bf16_bits_to_f32(xb).astype(np.float64) @ orc.bf16_bits_to_f32(wb).astype(np.float64).T
    assert rel_l2(yf, exact) <= 1e-6


def test_bf16_gemm_batched_src1(env):
    """src1 with ne2 > 1 (ggml broadcast of a 2-D weight over batches)."""
    tsk, orc = env
    rng = np.random.default_rng(12)
    wb = orc.f32_to_bf16_bits((rng.standard_normal((256, 512)) * 0.05).astype(np.float32))
    x = rng.standard_normal((3, 2, 50, 512)).astype(np.float32)
    y = tsk.mul_mat(tsk.bf16_to_device(wb), tsk.to_device(x))
    yref = orc.mul_mat(wb, x, a_type=orc.BF16)
    assert rel_l2(y.numpy(), yref) <= 1e-3
    # non-uniform slices: a strided view of src1 is handled slice by slice
    xd = tsk.to_device(x)
    xs = xd.view(0, (3, 2, 40, 512), xd.strides)
    y2 = tsk.mul_mat(tsk.bf16_to_device(wb), xs)
    yref2 = orc.mul_mat(wb, np.ascontiguousarray(x[:, :, :40]), a_type=orc.BF16)
    assert rel_l2(y2.numpy(), yref2) <= 1e-3


SHAPES_Q8 = [(1446, 1024, 3072), (1446, 1024, 1024), (1446, 1024, 4096), (1446, 4096, 1024),
             (77, 2048, 5120), (5, 96, 40), (512, 5120, 2048)]


@pytest.mark.parametrize("N,K,M", SHAPES_Q8)
def test_q8_0_gemm(env, N, K, M):
    """config 3 Q8_0 GEMMs: int8 values uniform in [-127,127], fp16 block scales."""
    tsk, orc = env
    rng = np.random.default_rng(N + K + M)
    blocks = np.zeros((M, K // 32, 34), np.uint8)
    qs = rng.integers(-127, 128, size=(M, K // 32, 32)).astype(np.int8)
    d = (np.abs(rng.standard_normal((M, K // 32))) * 0.02 / 127 + 1e-5).astype(np.float16)
    blocks[..., :2] = d.view(np.uint8).reshape(M, K // 32, 2)
    blocks[..., 2:] = qs.view(np.uint8)
    x = rng.standard_normal((N, K)).astype(np.float32)
    y = tsk.mul_mat(tsk.to_device(blocks), tsk.to_device(x), a_type=tsk.Q8_0)
    yref = orc.mul_mat(blocks, x, a_type=orc.Q8_0)
    assert rel_l2(y.numpy(), yref) <= 1e-3
    # exact integer block sums: the GPU differs from brute force by fp32 summation only
    exact = refmath.q8_0_matmul_exact(blocks, orc.quantize_q8_0(x, orc.Q8_CPU_SIMD))
    assert rel_l2(y.numpy(), exact) <= 1e-5
    # repacked weights give the same result bit for bit
    sp = tsk.q8_0_repack(tsk.to_device(blocks))
    y2 = tsk.mul_mat(sp, tsk.to_device(x), a_type=tsk.Q8_0_SPLIT)
    assert np.array_equal(y.numpy(), y2.numpy())


def test_q8_0_dequant_and_quant_bit_exact(env):
    tsk, orc = env
    rng = np.random.default_rng(13)
    w = (rng.standard_normal((300, 1024)) * 0.02).astype(np.float32)
    w[5, :32] = 0.0                                            # all-zero block: d = 0
    w[6, :32] = np.arange(32) - 15.5                          # exact .5 ties after scaling
    blocks = orc.quantize_q8_0(w, orc.Q8_CPU_SIMD)
    gpu_blocks = tsk.q8_0_quantize(tsk.to_device(w)).numpy()
    assert np.array_equal(gpu_blocks, blocks)
    deq = tsk.q8_0_dequantize(tsk.to_device(blocks)).numpy()
    assert np.array_equal(deq.view(np.uint32), orc.dequantize_q8_0(blocks).view(np.uint32))
    sp = tsk.q8_0_repack(tsk.to_device(blocks))
    deq2 = tsk.q8_0_dequantize(sp).numpy()
    assert np.array_equal(deq2.view(np.uint32), deq.view(np.uint32))
    g = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "q8_0.npz"))
    kat = tsk.q8_0_dequantize(tsk.to_device(np.ascontiguousarray(g["kat_blocks"][:, None, :])))
    assert np.array_equal(kat.numpy(), g["kat_deq"])


@pytest.mark.parametrize("cfg", [2, 5])
@pytest.mark.parametrize("N,K,M", [(512, 5120, 2048), (300, 4096, 1024), (77, 2176, 256), (130, 2176, 208),
                                   (1446, 1024, 3072)])
def test_q8_0_cooperative_matches_2x2_wave_kernel(env, N, K, M, cfg, monkeypatch):
    """Both cooperative Q8_0 tiles (cfg 2: 64 x 64, the T5 qkv / wi shape;
    cfg 5: 32 x 64, rows x tokens) stage block scales in 1024-k segments for
    long K (2176 and 5120: three and five segments, the last one partial);
    each output still sums its blocks in block order, so both equal the
    2 x 2-wave kernel bit for bit. M = 208 (M % 32 == 16) leaves cfg 5 a
    partial last row tile; N = 77 and 130 partial token tiles."""
    tsk, orc = env
    rng = np.random.default_rng(K + M)
    blocks = np.zeros((M, K // 32, 34), np.uint8)
    qs = rng.integers(-127, 128, size=(M, K // 32, 32)).astype(np.int8)
    d = (np.abs(rng.standard_normal((M, K // 32))) * 0.02 / 127 + 1e-5).astype(np.float16)
    blocks[..., :2] = d.view(np.uint8).reshape(M, K // 32, 2)
    blocks[..., 2:] = qs.view(np.uint8)
    x = tsk.to_device(rng.standard_normal((N, K)).astype(np.float32))
    sp = tsk.q8_0_repack(tsk.to_device(blocks))
    try:
        monkeypatch.setenv("TSK_Q8_CFG", str(cfg))
        tsk.init(0, reread=True)
        y = tsk.mul_mat(sp, x, a_type=tsk.Q8_0_SPLIT).numpy()
        monkeypatch.setenv("TSK_Q8_OLD", "1")
        tsk.init(0, reread=True)
        y_old = tsk.mul_mat(sp, x, a_type=tsk.Q8_0_SPLIT).numpy()
    finally:
        monkeypatch.delenv("TSK_Q8_OLD", raising=False)
        monkeypatch.delenv("TSK_Q8_CFG", raising=False)
        tsk.init(0, reread=True)
    assert np.array_equal(y, y_old)
