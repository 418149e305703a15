"""ctypes front end of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker that the HIP path is compared against
and the timed CPU baseline of bench.py. Nothing in the product imports it.

Arrays follow numpy C order, i.e. the reverse of ggml's ne[]: a ggml tensor
ne = [D, N, H, B] is a numpy array of shape (B, H, N, D). 16-bit float types
are passed as numpy float16 (F16) or as uint16 bit patterns (BF16).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q8_0, I32, BF16 = 0, 1, 8, 26, 30
Q8_CPU_SIMD, Q8_CPU_REF, Q8_GGUF_PY = 0, 1, 2


class TskTensor(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_size_t * 4), ("data", ctypes.c_void_p)]


class T5Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "d_model", "d_ff", "n_layers", "n_heads", "d_kv", "rel_buckets", "rel_max_dist",
        "weight_type", "max_tokens")] + [("eps", ctypes.c_float)]


class DitConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "hidden", "n_head", "head_dim", "depth", "fused_depth", "latent_dim", "text_seq",
        "mlp_hidden", "mlp_kind", "weight_type", "max_batch", "max_latent")] + \
        [(n, ctypes.c_float) for n in ("rope_theta", "t_max_period", "ln_eps", "qk_eps")]


class VaeConfig(ctypes.Structure):
    _fields_ = [("latent_dim", ctypes.c_int), ("channels", ctypes.c_int), ("out_channels", ctypes.c_int),
                ("c_mults", ctypes.c_int * 5), ("strides", ctypes.c_int * 5), ("max_latent", ctypes.c_int)]


class MMDitConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "hidden", "n_head", "head_dim", "depth", "fused_depth", "latent_dim", "text_seq", "clip_dim",
        "sync_dim", "t5_dim", "mlp_hidden", "max_batch", "max_latent", "max_clip", "max_sync")] + \
        [(n, ctypes.c_float) for n in ("rope_theta", "t_max_period")] + [("weight_type", ctypes.c_int)]


_lib = None


def build():
    subprocess.check_call(["make", "-s", "-C", HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER(TskTensor)
        L.orc_mul_mat.argtypes = [P, P, P, P]
        L.orc_flash_attn_ext.argtypes = [P, P, P, P, ctypes.c_float, ctypes.c_float,
                                         ctypes.c_float, ctypes.c_int, P]
        L.orc_rms_norm_mul.argtypes = [P, ctypes.c_void_p, ctypes.c_float, P]
        L.orc_norm.argtypes = [P, ctypes.c_float, P]
        L.orc_rope_ext.argtypes = [P, ctypes.c_void_p, ctypes.c_int, ctypes.c_float,
                                   ctypes.c_float, P]
        L.orc_quantize_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                        ctypes.c_int]
        L.orc_dequantize_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.orc_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.orc_fp32_to_fp16.restype = ctypes.c_uint16
        L.orc_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.orc_fp16_to_fp32.restype = ctypes.c_float
        L.orc_fp32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_fp32_to_bf16.restype = ctypes.c_uint16
        for nm in ("orc_fp32_to_fp16_row", "orc_fp16_to_fp32_row",
                   "orc_fp32_to_bf16_row", "orc_bf16_to_fp32_row"):
            getattr(L, nm).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_gelu_tanh.argtypes = [ctypes.c_float]
        L.orc_gelu_tanh.restype = ctypes.c_float
        L.orc_dit_create.argtypes = [ctypes.POINTER(DitConfig)]
        L.orc_dit_create.restype = ctypes.c_void_p
        L.orc_dit_destroy.argtypes = [ctypes.c_void_p]
        L.orc_dit_set_tensor_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_size_t]
        L.orc_dit_n_tensors.argtypes = [ctypes.c_void_p]
        L.orc_dit_tensor_info.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
                                          ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]
        L.orc_dit_set_tensor.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p,
                                         ctypes.c_int64]
        L.orc_dit_forward.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.orc_dit_sample.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                     ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int, ctypes.c_int]
        vp = ctypes.c_void_p
        L.orc_t5_bucket.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_t5_attention.argtypes = [vp, vp, vp, ctypes.c_int64, vp, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, vp]
        L.orc_t5_create.argtypes = [ctypes.POINTER(T5Config)]
        L.orc_t5_create.restype = vp
        L.orc_t5_destroy.argtypes = [vp]
        L.orc_t5_n_tensors.argtypes = [vp]
        L.orc_t5_tensor_info.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
                                         ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64),
                                         ctypes.POINTER(ctypes.c_int)]
        L.orc_t5_set_tensor.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_size_t]
        L.orc_t5_encode.argtypes = [vp, ctypes.c_int, vp, vp, vp]
        L.orc_t5_encode_range.argtypes = [vp, ctypes.c_int, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
        L.orc_im2col_1d.argtypes = [ctypes.c_int, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
        L.orc_conv1d.argtypes = [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P]
        L.orc_swiglu.argtypes = [vp, vp, vp, ctypes.c_int64]
        L.orc_conv_mlp_swiglu.argtypes = [P, P, P, P, P]
        L.orc_mmdit_create.argtypes = [ctypes.POINTER(MMDitConfig)]
        L.orc_mmdit_create.restype = vp
        L.orc_mmdit_destroy.argtypes = [vp]
        L.orc_mmdit_n_tensors.argtypes = [vp]
        L.orc_mmdit_tensor_info.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p),
                                            ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int)]
        L.orc_mmdit_set_tensor.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_int64]
        L.orc_mmdit_set_tensor_q8_0.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_size_t]
        L.orc_mmdit_set_type.argtypes = [vp, ctypes.c_char_p, ctypes.c_int]
        L.orc_mmdit_forward.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp, vp, ctypes.c_int, vp, ctypes.c_int, vp,
                                        vp, vp, vp, vp, ctypes.c_int, ctypes.c_int]
        L.orc_vae_create.argtypes = [ctypes.POINTER(VaeConfig)]
        L.orc_vae_create.restype = vp
        L.orc_vae_destroy.argtypes = [vp]
        L.orc_vae_n_tensors.argtypes = [vp]
        L.orc_vae_tensor_info.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int64)]
        L.orc_vae_set_tensor.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_int64]
        L.orc_vae_decode.argtypes = [vp, ctypes.c_int, vp, vp]
        L.orc_mmdit_stage_size.argtypes = [vp, ctypes.c_char_p]
        L.orc_mmdit_stage_size.restype = ctypes.c_int64
        L.orc_mmdit_stage.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_int64]
        L.orc_mmdit_sample.argtypes = [vp, ctypes.c_int, vp, ctypes.c_int, vp, ctypes.c_int, vp, vp, vp, vp,
                                       ctypes.c_int, ctypes.c_float, vp, vp, ctypes.c_int, ctypes.c_int]
        L.orc_mlp_swiglu.argtypes = [P, P, P, P, P]
        _lib = L
    return _lib


def set_threads(n):
    lib().orc_set_threads(int(n))


# ---------------------------------------------------------------- conversions
def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_fp32_to_fp16_row(x.ctypes.data, y.ctypes.data, x.size)
    return y


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().orc_fp16_to_fp32_row(h.ctypes.data, y.ctypes.data, h.size)
    return y


def f32_to_bf16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_fp32_to_bf16_row(x.ctypes.data, y.ctypes.data, x.size)
    return y


def bf16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().orc_bf16_to_fp32_row(h.ctypes.data, y.ctypes.data, h.size)
    return y


# ---------------------------------------------------------------- tensors
def tensor(arr, ttype):
    """tsk_tensor view of a C-contiguous numpy array (shape reversed to ne)."""
    assert arr.flags["C_CONTIGUOUS"]
    t = TskTensor()
    t.type = ttype
    shape = list(arr.shape)[::-1]
    strides = list(arr.strides)[::-1]
    if ttype == Q8_0:
        # arr is (rows, K/32, 34) uint8 -> ne = [K, rows]
        rows, nblk = arr.shape[0], arr.shape[1]
        shape = [nblk * 32, rows]
        strides = [34, nblk * 34]
    while len(shape) < 4:
        shape.append(1)
        strides.append(strides[-1] * (shape[-2] if len(shape) > 1 else 1))
    for i in range(4):
        t.ne[i] = shape[i]
        t.nb[i] = strides[i]
    t.data = arr.ctypes.data
    return t


def _ttype(arr, bf16):
    if arr.dtype == np.float32:
        return F32
    if arr.dtype == np.float16:
        return F16
    if arr.dtype == np.uint16 and bf16:
        return BF16
    raise TypeError(arr.dtype)


# ---------------------------------------------------------------- Q8_0
def gelu_tanh(x):
    """orc_gelu_tanh element by element (float32 in and out)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    f = lib().orc_gelu_tanh
    return np.array([f(float(v)) for v in x.ravel()], dtype=np.float32).reshape(x.shape)


def quantize_q8_0(x, mode=Q8_CPU_SIMD):
    """(..., K) float32 -> (rows, K/32, 34) uint8 ggml block_q8_0 bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[-1]
    rows = x.size // K
    out = np.empty((rows, K // 32, 34), dtype=np.uint8)
    lib().orc_quantize_q8_0(x.ctypes.data, out.ctypes.data, x.size, mode)
    return out


def dequantize_q8_0(blocks):
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    rows, nb = blocks.shape[0], blocks.shape[1]
    y = np.empty((rows, nb * 32), dtype=np.float32)
    lib().orc_dequantize_q8_0(blocks.ctypes.data, y.ctypes.data, rows * nb * 32)
    return y


# ---------------------------------------------------------------- ops
def mul_mat(a, b, bias=None, a_type=None):
    """ggml_mul_mat: a is (M, K) weights (F32/F16/BF16-bits or Q8_0 blocks),
    b is (..., N, K) float32 -> (..., N, M) float32."""
    a = np.ascontiguousarray(a)
    if a_type is None:
        a_type = _ttype(a, False)
    b = np.ascontiguousarray(b, dtype=np.float32)
    M = a.shape[0]
    out = np.empty(b.shape[:-1] + (M,), dtype=np.float32)
    ta, tb, td = tensor(a, a_type), tensor(b, F32), tensor(out, F32)
    tbias = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        tbias = ctypes.byref(tensor(bias, F32))
    rc = lib().orc_mul_mat(ctypes.byref(ta), ctypes.byref(tb), tbias, ctypes.byref(td))
    assert rc == 0, rc
    return out


def flash_attn_ext(q, k, v, mask=None, scale=0.125, max_bias=0.0, softcap=0.0,
                   vacc_f16=False, kv_bf16=False, q_bf16=False):
    """q (B,H,Nq,D), k/v (B,Hkv,Nkv,D) -> (B,Nq,H,D) float32 (ggml permuted)."""
    # keep the contiguous copies alive: tensors hold raw pointers
    q, k, v = (np.ascontiguousarray(a) for a in (q, k, v))
    B, H, Nq, D = q.shape
    out = np.empty((B, Nq, H, v.shape[-1]), dtype=np.float32)
    tq = tensor(q, _ttype(q, q_bf16))
    tk = tensor(k, _ttype(k, kv_bf16))
    tv = tensor(v, _ttype(v, kv_bf16))
    tm = None
    if mask is not None:
        mask = np.ascontiguousarray(mask)
        tm = ctypes.byref(tensor(mask, _ttype(mask, False)))
    td = tensor(out, F32)
    rc = lib().orc_flash_attn_ext(ctypes.byref(tq), ctypes.byref(tk), ctypes.byref(tv), tm,
                                  scale, max_bias, softcap, int(vacc_f16), ctypes.byref(td))
    assert rc == 0, rc
    return out


def rms_norm_mul(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    wp = None
    if w is not None:
        w = np.ascontiguousarray(w, dtype=np.float32)
        wp = w.ctypes.data
    rc = lib().orc_rms_norm_mul(ctypes.byref(tensor(x, F32)), wp, eps, ctypes.byref(tensor(out, F32)))
    assert rc == 0
    return out


def norm(x, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    rc = lib().orc_norm(ctypes.byref(tensor(x, F32)), eps, ctypes.byref(tensor(out, F32)))
    assert rc == 0
    return out


def rope_ext(x, pos, n_dims, freq_base=10000.0, freq_scale=1.0):
    """x (B, S, H, D) float32 (ggml ne [D, H, S, B]), pos int32 (S,)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    out = np.empty_like(x)
    rc = lib().orc_rope_ext(ctypes.byref(tensor(x, F32)), pos.ctypes.data, n_dims, freq_base,
                            freq_scale, ctypes.byref(tensor(out, F32)))
    assert rc == 0
    return out


# ---------------------------------------------------------------- convolution / SwiGLU
def conv_len(iw, kw, s0=1, p0=1, d0=1):
    return (iw + 2 * p0 - d0 * (kw - 1) - 1) // s0 + 1


def im2col_1d(x, kw, s0=1, p0=1, d0=1):
    """ggml_im2col 1-D: x (N, IC, IW) float32 -> (N, OW, IC*KW) float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    N, IC, IW = x.shape
    out = np.empty((N, conv_len(IW, kw, s0, p0, d0), IC * kw), dtype=np.float32)
    rc = lib().orc_im2col_1d(kw, ctypes.byref(tensor(x, F32)), s0, p0, d0, ctypes.byref(tensor(out, F32)))
    assert rc == 0, rc
    return out


def _kernel(w, w_type):
    """(OC, IC, KW) kernel values (float32, float16 or bf16 bits) -> tsk view."""
    w = np.ascontiguousarray(w)
    return w, tensor(w, w_type if w_type is not None else _ttype(w, False))


def conv1d(w, x, bias=None, s0=1, p0=1, d0=1, w_type=None):
    """conv_cl: w (OC, IC, KW) (ggml ne [KW, IC, OC]), x (B, IW, IC) float32
    channels fastest -> (B, OW, OC) float32."""
    w, tw = _kernel(w, w_type)
    x = np.ascontiguousarray(x, dtype=np.float32)
    B, IW, _ = x.shape
    out = np.empty((B, conv_len(IW, w.shape[2], s0, p0, d0), w.shape[0]), dtype=np.float32)
    tb = None
    if bias is not None:
        bias = np.ascontiguousarray(bias, dtype=np.float32)
        tb = ctypes.byref(tensor(bias, F32))
    rc = lib().orc_conv1d(ctypes.byref(tw), tb, ctypes.byref(tensor(x, F32)), s0, p0, d0,
                          ctypes.byref(tensor(out, F32)))
    assert rc == 0, rc
    return out


def swiglu(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty_like(a)
    lib().orc_swiglu(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size)
    return out


def conv_mlp_swiglu(w1, w3, w2, x, w_type=None):
    """convmlp: kernels (HID, IC, KW), (HID, IC, KW), (OC, HID, KW); x (B, IW, IC)."""
    (w1, t1), (w3, t3), (w2, t2) = (_kernel(w, w_type) for w in (w1, w3, w2))
    x = np.ascontiguousarray(x, dtype=np.float32)
    B, IW, _ = x.shape
    ow = conv_len(conv_len(IW, w1.shape[2]), w2.shape[2])
    out = np.empty((B, ow, w2.shape[0]), dtype=np.float32)
    rc = lib().orc_conv_mlp_swiglu(ctypes.byref(t1), ctypes.byref(t3), ctypes.byref(t2),
                                   ctypes.byref(tensor(x, F32)), ctypes.byref(tensor(out, F32)))
    assert rc == 0, rc
    return out


def mlp_swiglu(w1, w3, w2, x, w_type=None):
    """mlp: weights (HID, IC), (HID, IC), (OC, HID); x (..., IC) -> (..., OC)."""
    (w1, t1), (w3, t3), (w2, t2) = (_kernel(w, w_type) for w in (w1, w3, w2))
    x = np.ascontiguousarray(x, dtype=np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    out = np.empty((x2.shape[0], w2.shape[0]), dtype=np.float32)
    rc = lib().orc_mlp_swiglu(ctypes.byref(t1), ctypes.byref(t3), ctypes.byref(t2),
                              ctypes.byref(tensor(x2, F32)), ctypes.byref(tensor(out, F32)))
    assert rc == 0, rc
    return out.reshape(x.shape[:-1] + (w2.shape[0],))


# ---------------------------------------------------------------- MM-DiT
def dit_config(**kw):
    c = DitConfig(hidden=1024, n_head=16, head_dim=64, depth=21, fused_depth=14, latent_dim=64,
                  text_seq=77, mlp_hidden=4096, mlp_kind=0, weight_type=BF16, max_batch=2,
                  max_latent=646, rope_theta=10000.0, t_max_period=1.0, ln_eps=1e-5, qk_eps=1e-6)
    for k_, v_ in kw.items():
        setattr(c, k_, v_)
    return c


class OracleDiT:
    def __init__(self, cfg):
        self.cfg = cfg
        self.h = lib().orc_dit_create(ctypes.byref(cfg))

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_dit_destroy(self.h)
            self.h = None

    def tensors(self):
        out = []
        for i in range(lib().orc_dit_n_tensors(self.h)):
            nm, a, b = ctypes.c_char_p(), ctypes.c_int64(), ctypes.c_int64()
            lib().orc_dit_tensor_info(self.h, i, ctypes.byref(nm), ctypes.byref(a), ctypes.byref(b))
            out.append((nm.value.decode(), (a.value, b.value, 1, 1)))
        return out

    def set_tensor(self, name, arr):
        arr = np.ascontiguousarray(arr, dtype=np.float32)
        rc = lib().orc_dit_set_tensor(self.h, name.encode(), arr.ctypes.data, arr.size)
        assert rc == 0, (name, rc)

    def set_tensor_q8_0(self, name, blocks):
        """ggml Q8_0 blocks (uint8, 34 bytes per 32 values) of a Q8_0 block projection"""
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        rc = lib().orc_dit_set_tensor_q8_0(self.h, name.encode(), blocks.ctypes.data, blocks.nbytes)
        assert rc == 0, (name, rc)

    def forward(self, latent, t, text, act_bf16=True, kv_f16=True):
        latent = np.ascontiguousarray(latent, dtype=np.float32)
        t = np.ascontiguousarray(t, dtype=np.float32)
        text = np.ascontiguousarray(text, dtype=np.float32)
        B, T, L = latent.shape
        flow = np.empty((B, T, L), dtype=np.float32)
        rc = lib().orc_dit_forward(self.h, B, T, latent.ctypes.data, t.ctypes.data,
                                   text.ctypes.data, flow.ctypes.data, int(act_bf16), int(kv_f16))
        assert rc == 0
        return flow

    def sample(self, noise, text_cond, text_uncond, steps=24, cfg_scale=5.0, act_bf16=True,
               kv_f16=True):
        noise = np.ascontiguousarray(noise, dtype=np.float32)
        text_cond = np.ascontiguousarray(text_cond, dtype=np.float32)
        text_uncond = np.ascontiguousarray(text_uncond, dtype=np.float32)
        T, L = noise.shape
        out = np.empty((T, L), dtype=np.float32)
        flow0 = np.empty((T, L), dtype=np.float32)
        rc = lib().orc_dit_sample(self.h, T, noise.ctypes.data, text_cond.ctypes.data,
                                  text_uncond.ctypes.data, steps, cfg_scale, out.ctypes.data,
                                  flow0.ctypes.data, int(act_bf16), int(kv_f16))
        assert rc == 0
        return out, flow0


# ---------------------------------------------------------------- the reference's MM-DiT graph
def mmdit_config(**kw):
    """the reference's sizes (src/mmdit.h:17-22) with capacities for 30 s"""
    c = MMDitConfig(hidden=1024, n_head=16, head_dim=64, depth=21, fused_depth=14, latent_dim=64, text_seq=77,
                    clip_dim=1024, sync_dim=768, t5_dim=2048, mlp_hidden=2816, max_batch=2, max_latent=646,
                    max_clip=240, max_sync=720, rope_theta=10000.0, t_max_period=1.0, weight_type=BF16)
    for k_, v_ in kw.items():
        setattr(c, k_, v_)
    return c


class OracleMMDiT:
    """ts_dit::forward / ::sample restated (tsk_oracle_mmdit.c). Arrays in
    numpy C order of the ggml layouts: latent (B, L, T), clip (B, S_c, clip_dim),
    sync (B, S_s, sync_dim), text (B, 77, clip_dim), t5 (B, 77, t5_dim),
    g (B, clip_dim) -> flow (B, T, L)."""

    def __init__(self, cfg):
        self.cfg = cfg
        self.h = lib().orc_mmdit_create(ctypes.byref(cfg))

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_mmdit_destroy(self.h)
            self.h = None

    def tensors(self):
        """[(name, ggml ne (3), type)]"""
        out = []
        for i in range(lib().orc_mmdit_n_tensors(self.h)):
            nm, ne, ty = ctypes.c_char_p(), (ctypes.c_int64 * 3)(), ctypes.c_int()
            assert lib().orc_mmdit_tensor_info(self.h, i, ctypes.byref(nm), ne, ctypes.byref(ty)) == 0
            out.append((nm.value.decode(), tuple(ne), ty.value))
        return out

    def set_tensor(self, name, arr):
        arr = np.ascontiguousarray(arr, dtype=np.float32)
        rc = lib().orc_mmdit_set_tensor(self.h, name.encode(), arr.ctypes.data, arr.size)
        assert rc == 0, (name, rc)

    def set_tensor_q8_0(self, name, blocks):
        """Q8_0 blocks (bytes / uint8 array) as a GGUF file holds them"""
        b = np.ascontiguousarray(np.frombuffer(bytes(blocks), np.uint8))
        rc = lib().orc_mmdit_set_tensor_q8_0(self.h, name.encode(), b.ctypes.data, b.size)
        assert rc == 0, (name, rc)

    def set_type(self, name, type_id):
        rc = lib().orc_mmdit_set_type(self.h, name.encode(), int(type_id))
        assert rc == 0, (name, rc)

    @staticmethod
    def _c(a):
        return np.ascontiguousarray(a, dtype=np.float32)

    def forward(self, latent, t, clip, sync, text, t5, g, act_bf16=True, kv_f16=True):
        latent, t, clip, sync, text, t5, g = (self._c(a) for a in (latent, t, clip, sync, text, t5, g))
        B, L, T = latent.shape
        flow = np.empty((B, T, L), dtype=np.float32)
        rc = lib().orc_mmdit_forward(self.h, B, T, latent.ctypes.data, t.ctypes.data, clip.shape[1],
                                     clip.ctypes.data, sync.shape[1], sync.ctypes.data, text.ctypes.data,
                                     t5.ctypes.data, g.ctypes.data, flow.ctypes.data, int(act_bf16), int(kv_f16))
        assert rc == 0, rc
        return flow

    def stage(self, name):
        """a stage output of the last forward (flat, batch rows concatenated)"""
        n = lib().orc_mmdit_stage_size(self.h, name.encode())
        assert n >= 0, name
        out = np.empty(n, np.float32)
        assert lib().orc_mmdit_stage(self.h, name.encode(), out.ctypes.data, n) == 0
        return out

    def sample(self, noise, clip, sync, text, t5, g, steps=24, cfg_scale=5.0, act_bf16=True, kv_f16=True):
        """noise / out / flow0 (L, T)"""
        noise, clip, sync, text, t5, g = (self._c(a) for a in (noise, clip, sync, text, t5, g))
        L, T = noise.shape
        out = np.empty((L, T), dtype=np.float32)
        flow0 = np.empty((L, T), dtype=np.float32)
        rc = lib().orc_mmdit_sample(self.h, T, noise.ctypes.data, clip.shape[0], clip.ctypes.data, sync.shape[0],
                                    sync.ctypes.data, text.ctypes.data, t5.ctypes.data, g.ctypes.data, steps,
                                    cfg_scale, out.ctypes.data, flow0.ctypes.data, int(act_bf16), int(kv_f16))
        assert rc == 0, rc
        return out, flow0


# ---------------------------------------------------------------- Oobleck VAE decoder
def vae_config(**kw):
    """the reference's decoder (convert/convert_vae.py:60-66)"""
    c = VaeConfig(latent_dim=64, channels=128, out_channels=2, max_latent=646)
    c.c_mults[:] = kw.pop("c_mults", [1, 2, 4, 8, 16])
    c.strides[:] = kw.pop("strides", [2, 4, 4, 8, 8])
    for k_, v_ in kw.items():
        setattr(c, k_, v_)
    return c


class OracleVae:
    """ts_vae::decode restated (tsk_oracle_vae.c): latent (L, T) -> audio (C_out, T * hop)"""

    def __init__(self, cfg):
        self.cfg = cfg
        self.hop = int(np.prod(list(cfg.strides)))
        self.h = lib().orc_vae_create(ctypes.byref(cfg))

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_vae_destroy(self.h)
            self.h = None

    def tensors(self):
        out = []
        for i in range(lib().orc_vae_n_tensors(self.h)):
            nm, ne = ctypes.c_char_p(), (ctypes.c_int64 * 3)()
            assert lib().orc_vae_tensor_info(self.h, i, ctypes.byref(nm), ne) == 0
            out.append((nm.value.decode(), tuple(ne)))
        return out

    def set_tensor(self, name, arr):
        arr = np.ascontiguousarray(arr, dtype=np.float32)
        assert lib().orc_vae_set_tensor(self.h, name.encode(), arr.ctypes.data, arr.size) == 0, name

    def decode(self, latent):
        latent = np.ascontiguousarray(latent, dtype=np.float32)
        L, T = latent.shape
        audio = np.empty((self.cfg.out_channels, T * self.hop), np.float32)
        assert lib().orc_vae_decode(self.h, T, latent.ctypes.data, audio.ctypes.data) == 0
        return audio


# ---------------------------------------------------------------- T5 encoder (config 4)
def t5_config(**kw):
    c = T5Config(d_model=2048, d_ff=5120, n_layers=24, n_heads=32, d_kv=64, rel_buckets=32,
                 rel_max_dist=128, weight_type=Q8_0, max_tokens=512, eps=1e-6)
    for k_, v_ in kw.items():
        setattr(c, k_, v_)
    return c


def t5_bucket(rel, num_buckets=32, max_dist=128):
    """relative-position bucket of src/t5_encoder.cpp:14-26"""
    return lib().orc_t5_bucket(int(rel), int(num_buckets), int(max_dist))


def t5_attention_mask(rel_bias, ids, num_buckets=32, max_dist=128):
    """[H][n][n] f32 additive mask: rel_bias[bucket(k - q)][h] + (-inf where ids[k] == 0)."""
    rel_bias = np.asarray(rel_bias, dtype=np.float32)       # (buckets, H)
    n = len(ids)
    table = np.array([t5_bucket(r, num_buckets, max_dist) for r in range(-(n - 1), n)], dtype=np.int64)
    rel = np.arange(n)[None, :] - np.arange(n)[:, None]    # k - q
    bk = table[rel + (n - 1)]                               # (q, k)
    m = rel_bias[bk].transpose(2, 0, 1).astype(np.float32)  # (H, q, k)
    pad = np.where(np.asarray(ids) != 0, 0.0, -np.inf).astype(np.float32)
    return np.ascontiguousarray(m + pad[None, None, :])


def t5_attention(q, k, v, mask):
    """q/k/v (n, H, D) f32 rows, mask (H, n, n) -> (n, H, D): the reference's
    mul_mat / add / soft_max / mul_mat chain (src/t5_encoder.cpp:68-75)."""
    q, k, v, mask = (np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v, mask))
    n, H, D = q.shape
    out = np.empty((n, H, D), np.float32)
    rc = lib().orc_t5_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data, H * D, mask.ctypes.data,
                                n, H, D, out.ctypes.data)
    assert rc == 0
    return out


class OracleT5:
    def __init__(self, cfg):
        self.cfg = cfg
        self.h = lib().orc_t5_create(ctypes.byref(cfg))

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_t5_destroy(self.h)
            self.h = None

    def tensors(self):
        out = []
        for i in range(lib().orc_t5_n_tensors(self.h)):
            nm, a, b, t = ctypes.c_char_p(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int()
            lib().orc_t5_tensor_info(self.h, i, ctypes.byref(nm), ctypes.byref(a), ctypes.byref(b),
                                     ctypes.byref(t))
            out.append((nm.value.decode(), (a.value, b.value, 1, 1), t.value))
        return out

    def set_tensor(self, name, data):
        data = np.ascontiguousarray(data)
        rc = lib().orc_t5_set_tensor(self.h, name.encode(), data.ctypes.data, data.nbytes)
        assert rc == 0, (name, rc)

    def encode(self, x, ids, layers=None, final_norm=True):
        """layers = (begin, end) runs only those layers (default: all)"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty_like(x)
        b, e = layers if layers is not None else (0, self.cfg.n_layers)
        rc = lib().orc_t5_encode_range(self.h, x.shape[0], x.ctypes.data, ids.ctypes.data, b, e,
                                       int(final_norm), out.ctypes.data)
        assert rc == 0
        return out
