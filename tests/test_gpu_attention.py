"""flash_attn_ext on gfx950 through the C ABI vs the oracle (ggml-cpu
semantics, oracle/tsk_oracle.c). Tolerances (rel-L2): fp32 attention <= 1e-5,
16-bit attention <= 1e-3."""
import numpy as np
import pytest

from conftest import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def env(orc):
    from __graft_entry__ import ensure_built, load_tsk
    ensure_built()
    tsk = load_tsk()
    tsk.init(0)
    return tsk, orc


@pytest.mark.parametrize("B,H,N", [(2, 16, 271), (1, 16, 77), (2, 8, 1), (1, 2, 65), (2, 16, 194), (2, 16, 646)])
def test_f32_attention(env, B, H, N):
    """config 1: F32 joint attention, scale 1/8, no mask (rel-L2 <= 1e-5). Up to 256
    workgroups of 64 query rows run two key ranges per workgroup (N = 65: the second
    range has only masked keys; 271: ranges of 3 and 2 tiles); N = 646 at B = 2 runs one."""
    tsk, orc = env
    rng = np.random.default_rng(1234 + N)
    q, k, v = (rng.standard_normal((B, H, N, 64)).astype(np.float32) for _ in range(3))
    o = tsk.flash_attn_ext(*(tsk.to_device(a) for a in (q, k, v)), scale=0.125)
    ref = orc.flash_attn_ext(q, k, v, scale=0.125)
    assert rel_l2(o.numpy(), ref) <= 1e-5


@pytest.mark.parametrize("B,H,N", [(1, 16, 420), (1, 16, 1040), (1, 16, 194), (1, 16, 646),
                                   (2, 16, 271), (1, 8, 77), (2, 16, 1040)])
def test_reference_types_f32q_f16kv(env, B, H, N):
    """the node mmdit.cpp:88-92 emits: Q F32, K/V cast to F16, prec F32; at
    B = 2, N = 1040 (the graph's 30 s joint attention) on the 2 x 5 launch
    shape the rule picks there."""
    tsk, orc = env
    rng = np.random.default_rng(N)
    q = rng.standard_normal((B, H, N, 64)).astype(np.float32)
    k = rng.standard_normal((B, H, N, 64)).astype(np.float16)
    v = rng.standard_normal((B, H, N, 64)).astype(np.float16)
    o = tsk.flash_attn_ext(tsk.to_device(q), tsk.to_device(k), tsk.to_device(v), scale=0.125)
    ref = orc.flash_attn_ext(q, k, v, scale=0.125)
    assert rel_l2(o.numpy(), ref) <= 1e-3


@pytest.mark.parametrize("N", [723, 271, 33])
def test_bf16_attention_config3(env, N):
    """config 3: bf16 Q/K/V after QK-RMSNorm and RoPE on the 646 latent positions."""
    tsk, orc = env
    rng = np.random.default_rng(99 + N)
    B, H = 2, 16
    x = [rng.standard_normal((B, N, H, 64)).astype(np.float32) for _ in range(3)]
    w = np.ones(64, np.float32)
    nlat = min(646, N)
    pos = np.arange(nlat, dtype=np.int32)
    qk = []
    for t in x[:2]:
        t = orc.rms_norm_mul(t, w, 1e-6)
        t[:, :nlat] = orc.rope_ext(np.ascontiguousarray(t[:, :nlat]), pos, 64)
        qk.append(t)
    bits = [orc.f32_to_bf16_bits(np.ascontiguousarray(t.transpose(0, 2, 1, 3))) for t in (qk[0], qk[1], x[2])]
    o = tsk.flash_attn_ext(*(tsk.bf16_to_device(b) for b in bits), scale=0.125)
    ref = orc.flash_attn_ext(*bits, scale=0.125, kv_bf16=True, q_bf16=True)
    assert rel_l2(o.numpy(), ref) <= 1e-3
    ob = tsk.flash_attn_ext(*(tsk.bf16_to_device(b) for b in bits), scale=0.125, out_dtype="bf16")
    assert rel_l2(orc.bf16_bits_to_f32(ob.numpy()), ref) <= 5e-3


def test_mask_gqa_softcap_alibi(env):
    """T5-style additive per-head bias + pad mask (config 4 path), GQA, softcap, ALiBi."""
    tsk, orc = env
    rng = np.random.default_rng(4)
    B, H, Hkv, N = 1, 8, 4, 130
    q = rng.standard_normal((B, H, N, 64)).astype(np.float32)
    k = rng.standard_normal((B, Hkv, N, 64)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, N, 64)).astype(np.float16)
    mask = rng.standard_normal((1, H, N, N)).astype(np.float16)
    mask[..., N - 20:] = -np.inf                                   # padded keys
    dev = tsk.to_device
    o = tsk.flash_attn_ext(dev(q), dev(k), dev(v), mask=dev(mask), scale=1.0)
    ref = orc.flash_attn_ext(q, k, v, mask=mask, scale=1.0)
    assert rel_l2(o.numpy(), ref) <= 1e-3
    o = tsk.flash_attn_ext(dev(q), dev(k), dev(v), mask=dev(mask), scale=0.125, max_bias=8.0, softcap=30.0)
    ref = orc.flash_attn_ext(q, k, v, mask=mask, scale=0.125, max_bias=8.0, softcap=30.0)
    assert rel_l2(o.numpy(), ref) <= 1e-3


def test_fully_masked_rows_and_ragged_kv(env):
    tsk, orc = env
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 2, 20, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 37, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 37, 64)).astype(np.float32)
    mask = np.zeros((1, 1, 32, 37), np.float16)
    mask[0, 0, 3, :] = -np.inf
    dev = tsk.to_device
    o = tsk.flash_attn_ext(dev(q), dev(k), dev(v), mask=dev(mask)).numpy()
    ref = orc.flash_attn_ext(q, k, v, mask=mask)
    assert np.all(np.isfinite(o)) and np.all(o[0, 3] == 0)
    assert rel_l2(o, ref) <= 1e-5


def test_strided_views_and_determinism(env):
    """q/k/v as permuted views of one qkv buffer (no copies), run twice bit-equal."""
    tsk, orc = env
    rng = np.random.default_rng(6)
    qkv = rng.standard_normal((2, 3, 16, 100, 64)).astype(np.float32)   # ggml ne [64,100,16,3,2]
    t = tsk.to_device(qkv)
    q, k, v = t.select(1, 0), t.select(1, 1), t.select(1, 2)
    o1 = tsk.flash_attn_ext(q, k, v).numpy()
    o2 = tsk.flash_attn_ext(q, k, v).numpy()
    assert np.array_equal(o1, o2)
    ref = orc.flash_attn_ext(qkv[:, 0], qkv[:, 1], qkv[:, 2])
    assert rel_l2(o1, ref) <= 1e-5


@pytest.mark.parametrize("kv,N", [("f16", 723), ("f16", 130), ("bf16", 723), ("bf16", 61)])
@pytest.mark.parametrize("v_offset", [0, 8])
def test_fast_path_permuted_views(env, kv, N, v_offset):
    """16-bit K/V as the permuted views ggml hands over (storage [B][N][H][64]:
    the key-row stride is H * 128 bytes, not one row), N not a multiple of 64
    (the last tile's K rows past N read as zeros through the buffer range and are
    masked), sizes on the 4 x 3 / 2 x 4 and 4 x 1 launch shapes, V at the start of
    its buffer or 16 bytes into it; a V 2 bytes off 16-byte alignment is refused
    on the host (TSK_ERR_ALIGN) before any launch."""
    tsk, orc = env
    rng = np.random.default_rng(7 * N + v_offset)
    B, H = 2, 16
    q = rng.standard_normal((B, N, H, 64)).astype(np.float32)
    kf = rng.standard_normal((B, N, H, 64)).astype(np.float32)
    vf = rng.standard_normal((B, N, H, 64)).astype(np.float32)
    perm = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))   # (B, H, N, 64)
    st = (N * H * 64, 64, H * 64, 1)                                 # element strides of the permuted view
    if kv == "f16":
        kb, vb = kf.astype(np.float16), vf.astype(np.float16)
        kd = tsk.to_device(kb)
        vbuf = tsk.DeviceArray((B * N * H * 64 + 16,), "f16")
        vhost = np.zeros(B * N * H * 64 + 16, np.float16)
        vhost[v_offset:v_offset + vb.size] = vb.ravel()
        qd = tsk.to_device(q)
        ref = orc.flash_attn_ext(perm(q), perm(kb), perm(vb), scale=0.125)
    else:
        qbits, kbits, vbits = (orc.f32_to_bf16_bits(a) for a in (q, kf, vf))
        kd = tsk.bf16_to_device(kbits)
        vbuf = tsk.DeviceArray((B * N * H * 64 + 16,), "bf16")
        vhost = np.zeros(B * N * H * 64 + 16, np.uint16)
        vhost[v_offset:v_offset + vbits.size] = vbits.ravel()
        qd = tsk.bf16_to_device(qbits)
        ref = orc.flash_attn_ext(perm(qbits), perm(kbits), perm(vbits), scale=0.125, kv_bf16=True, q_bf16=True)
    import ctypes
    tsk._hipcheck(tsk.hip().hipMemcpy(ctypes.c_void_p(vbuf.ptr), ctypes.c_void_p(vhost.ctypes.data), vhost.nbytes, 1),
                  "hipMemcpy H2D")
    qv = qd.view(0, (B, H, N, 64), st)
    kvw = kd.view(0, (B, H, N, 64), st)
    vv = vbuf.view(v_offset, (B, H, N, 64), st)
    o1 = tsk.flash_attn_ext(qv, kvw, vv, scale=0.125).numpy()
    o2 = tsk.flash_attn_ext(qv, kvw, vv, scale=0.125).numpy()
    assert np.array_equal(o1, o2)
    assert rel_l2(o1, ref) <= 1e-3
    with pytest.raises(tsk.TskError, match="ALIGN"):
        tsk.flash_attn_ext(qv, kvw, vbuf.view(v_offset + 1, (B, H, N, 64), st), scale=0.125)
