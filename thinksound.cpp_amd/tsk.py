"""Python front end of libtsk.so (ctypes over the C ABI in include/tsk/tsk.h).

Mirrors the ggml operator surface that src/mmdit.cpp drives for the MM-DiT
hot path -- mul_mat, flash_attn_ext, rms_norm*w, rope_ext, norm -- plus the
ts_dit driver (load / forward / sample, src/mmdit.h:9-42). Device tensors are
DeviceArrays allocated through the same HIP runtime libtsk.so links (no
second runtime in the process); shapes are numpy order, i.e. the reverse of
ggml's ne[] (a ggml [D, N, H, B] tensor has shape (B, H, N, D)). Errors raise
TskError with the library's status and message; nothing falls back to a CPU
path: if libtsk.so is missing, load() raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libtsk.so")

F32, F16, Q8_0, I32, BF16, Q8_0_SPLIT = 0, 1, 8, 26, 30, 0x1008
PREC_DEFAULT, PREC_F32 = 0, 10
ROPE_NORMAL = 0
OP_MUL_MAT, OP_FLASH_ATTN_EXT, OP_RMS_NORM_MUL, OP_ROPE_EXT, OP_NORM, OP_IM2COL, OP_CONV1D = 1, 2, 3, 4, 5, 6, 7
OP_CONV_MLP_SWIGLU, OP_MLP_SWIGLU, OP_RMS_NORM_Q8_0 = 8, 9, 10
STATUS = {0: "TSK_OK", -1: "TSK_ERR_INVALID_ARG", -2: "TSK_ERR_TYPE", -3: "TSK_ERR_SHAPE",
          -4: "TSK_ERR_STRIDE", -5: "TSK_ERR_ALIGN", -6: "TSK_ERR_UNSUPPORTED",
          -7: "TSK_ERR_NOT_INIT", -8: "TSK_ERR_HIP", -9: "TSK_ERR_NOMEM"}


class TskError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"{STATUS.get(status, status)}: {msg}")
        self.status = status


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


def load():
    """Load libtsk.so (built by __graft_entry__.build()); raise if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER(TskTensor)
    vp, f, i = ctypes.c_void_p, ctypes.c_float, ctypes.c_int
    sig = {
        "tsk_init": ([i], i), "tsk_shutdown": ([], i),
        "tsk_status_string": ([i], ctypes.c_char_p), "tsk_last_error": ([], ctypes.c_char_p),
        "tsk_version": ([], ctypes.c_char_p),
        "tsk_mul_mat": ([P, P, P, P, vp], i),
        "tsk_mul_mat_noalloc": ([P, P, P, P, vp], i),
        "tsk_flash_attn_ext": ([P, P, P, P, f, f, f, i, P, vp], i),
        "tsk_rms_norm_mul": ([P, P, f, P, vp], i),
        "tsk_t5_attention": ([P, P, P, P, vp, f, P, vp], i),
        "tsk_rms_norm_q8_0": ([P, P, f, P, vp], i),
        "tsk_norm": ([P, f, P, vp], i),
        "tsk_rope_ext": ([P, P, i, i, f, f, f, f, P, vp], i),
        "tsk_qk_norm_rope": ([P, P, P, f, i, f, f, P, vp], i),
        "tsk_q8_0_quantize": ([P, P, vp], i), "tsk_q8_0_dequantize": ([P, P, vp], i),
        "tsk_q8_0_repack": ([P, P, vp], i),
        "tsk_q8_0_split_nbytes": ([ctypes.c_int64, ctypes.c_int64], ctypes.c_size_t),
        "tsk_supports_op": ([i, ctypes.POINTER(P), i, P], i),
        "tsk_workspace_size": ([i, ctypes.POINTER(P), i, P, ctypes.POINTER(ctypes.c_size_t)], i),
        "tsk_set_workspace": ([vp, vp, ctypes.c_size_t], i),
        "tsk_release_workspace": ([vp], i),
        "tsk_im2col_1d": ([P, P, i, i, i, P, vp], i),
        "tsk_conv1d": ([P, P, P, i, i, i, P, vp], i),
        "tsk_conv1d_pack_weight": ([P, P, vp], i),
        "tsk_swiglu": ([P, P, P, vp], i),
        "tsk_conv_mlp_swiglu": ([P, P, P, P, P, vp], i),
        "tsk_mlp_swiglu": ([P, P, P, P, P, vp], i),
        "tsk_t5_default_config": ([ctypes.POINTER(T5Config)], None),
        "tsk_t5_create": ([ctypes.POINTER(T5Config), ctypes.POINTER(vp)], i),
        "tsk_t5_destroy": ([vp], None),
        "tsk_t5_n_tensors": ([vp], i),
        "tsk_t5_tensor_info": ([vp, i, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int64),
                                ctypes.POINTER(ctypes.c_int)], i),
        "tsk_t5_set_tensor": ([vp, ctypes.c_char_p, vp, ctypes.c_size_t], i),
        "tsk_t5_encode": ([vp, i, vp, vp, vp, vp], i),
        "tsk_t5_encode_device": ([vp, i, vp, vp, vp, vp], i),
        "tsk_t5_encode_range": ([vp, i, vp, vp, i, i, i, vp, vp], i),
        "tsk_t5_encode_layers": ([vp, i, vp, vp, i, i, i, vp, vp], i),
        "tsk_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(vp)], i),
        "tsk_gguf_close": ([vp], None),
        "tsk_gguf_n_tensors": ([vp], i),
        "tsk_gguf_tensor_info": ([vp, i, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int64),
                                  ctypes.POINTER(ctypes.c_int)], i),
        "tsk_gguf_find_tensor": ([vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int)], i),
        "tsk_gguf_read_tensor": ([vp, ctypes.c_char_p, i, vp, ctypes.c_size_t], i),
        "tsk_gguf_get_u32": ([vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)], i),
        "tsk_gguf_get_f32": ([vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)], i),
        "tsk_gguf_get_str": ([vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)], i),
        "tsk_dit_config_from_gguf": ([vp, ctypes.POINTER(DitConfig)], i),
        "tsk_dit_load_gguf": ([vp, vp], i),
        "tsk_t5_config_from_gguf": ([vp, ctypes.POINTER(T5Config)], i),
        "tsk_t5_load_gguf": ([vp, vp], i),
        "tsk_dit_default_config": ([ctypes.POINTER(DitConfig)], None),
        "tsk_dit_create": ([ctypes.POINTER(DitConfig), ctypes.POINTER(vp)], i),
        "tsk_dit_destroy": ([vp], None),
        "tsk_dit_n_tensors": ([vp], i),
        "tsk_dit_tensor_info": ([vp, i, ctypes.POINTER(ctypes.c_char_p),
                                 ctypes.POINTER(ctypes.c_int64)], i),
        "tsk_dit_set_tensor": ([vp, ctypes.c_char_p, vp, ctypes.c_int64], i),
        "tsk_dit_set_tensor_q8_0": ([vp, ctypes.c_char_p, vp, ctypes.c_size_t], i),
        "tsk_dit_tensor_type": ([vp, i], i),
        "tsk_dit_forward": ([vp, i, i, vp, vp, vp, vp, vp], i),
        "tsk_dit_forward_device": ([vp, i, i, vp, vp, vp, vp, vp], i),
        "tsk_dit_sample": ([vp, i, vp, vp, vp, i, f, vp, vp, vp], i),
        "tsk_mmdit_default_config": ([ctypes.POINTER(MMDitConfig)], None),
        "tsk_mmdit_create": ([ctypes.POINTER(MMDitConfig), ctypes.POINTER(vp)], i),
        "tsk_mmdit_destroy": ([vp], None),
        "tsk_mmdit_n_tensors": ([vp], i),
        "tsk_mmdit_tensor_info": ([vp, i, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int64)], i),
        "tsk_mmdit_tensor_type": ([vp, i], i),
        "tsk_mmdit_set_tensor": ([vp, ctypes.c_char_p, vp, ctypes.c_int64], i),
        "tsk_mmdit_set_tensor_q8_0": ([vp, ctypes.c_char_p, vp, ctypes.c_size_t], i),
        "tsk_mmdit_config_from_gguf": ([vp, ctypes.POINTER(MMDitConfig)], i),
        "tsk_mmdit_create_from_gguf": ([vp, ctypes.POINTER(MMDitConfig), ctypes.POINTER(vp)], i),
        "tsk_mmdit_load_gguf": ([vp, vp], i),
        "tsk_mmdit_forward": ([vp, i, i, vp, vp, i, vp, i, vp, vp, vp, vp, vp, vp], i),
        "tsk_mmdit_sample": ([vp, i, vp, i, vp, i, vp, vp, vp, vp, i, f, vp, vp, vp], i),
        "tsk_mmdit_forward_device": ([vp, i, i, vp, vp, i, vp, i, vp, vp, vp, vp, vp, vp], i),
        "tsk_mmdit_debug": ([vp, i], i),
        "tsk_mmdit_debug_size": ([vp, ctypes.c_char_p], ctypes.c_int64),
        "tsk_mmdit_debug_get": ([vp, ctypes.c_char_p, vp, ctypes.c_int64], i),
        "tsk_vae_default_config": ([ctypes.POINTER(VaeConfig)], None),
        "tsk_vae_create": ([ctypes.POINTER(VaeConfig), ctypes.POINTER(vp)], i),
        "tsk_vae_destroy": ([vp], None),
        "tsk_vae_n_tensors": ([vp], i),
        "tsk_vae_tensor_info": ([vp, i, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int64)], i),
        "tsk_vae_set_tensor": ([vp, ctypes.c_char_p, vp, ctypes.c_int64], i),
        "tsk_vae_hop": ([vp], i),
        "tsk_vae_decode": ([vp, i, vp, vp, ctypes.POINTER(ctypes.c_int64), vp], i),
        "tsk_vae_decode_device": ([vp, i, vp, vp, vp], i),
        "tsk_dit_timing": ([vp, i], i),
        "tsk_dit_timing_read": ([vp, i, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64),
                                 ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)], i),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def check(rc):
    if rc != 0:
        raise TskError(rc, load().tsk_last_error().decode())
    return rc


_initialised = False


def init(device=0, reread=False):
    """tsk_init once per process; reread=True calls it again (it re-reads the
    TSK_* launch-shape overrides from the environment)."""
    global _initialised
    if not _initialised or reread:
        check(load().tsk_init(device))
        _initialised = True


# ---------------------------------------------------------------- device memory
# The HIP runtime libtsk.so links (resolved by soname once libtsk is loaded),
# so buffers, streams and events all live in the same runtime as the kernels.
_hip = None
DTYPES = {"f32": (F32, 4, "float32"), "f16": (F16, 2, "float16"), "bf16": (BF16, 2, "uint16"),
          "i32": (I32, 4, "int32"), "u8": (-1, 1, "uint8")}


def hip():
    global _hip
    if _hip is None:
        load()
        H = ctypes.CDLL("libamdhip64.so.7")
        vp, sz, i = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        for nm, args in {"hipMalloc": [ctypes.POINTER(vp), sz], "hipFree": [vp],
                         "hipMemcpy": [vp, vp, sz, i], "hipMemcpyAsync": [vp, vp, sz, i, vp],
                         "hipMemset": [vp, i, sz], "hipDeviceSynchronize": [],
                         "hipStreamSynchronize": [vp], "hipEventCreate": [ctypes.POINTER(vp)],
                         "hipStreamCreate": [ctypes.POINTER(vp)], "hipStreamDestroy": [vp],
                         "hipEventDestroy": [vp], "hipEventRecord": [vp, vp],
                         "hipEventSynchronize": [vp],
                         "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
                         "hipStreamBeginCapture": [vp, i], "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
                         "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, vp, sz],
                         "hipGraphLaunch": [vp, vp], "hipGraphExecDestroy": [vp],
                         "hipGraphDestroy": [vp]}.items():
            getattr(H, nm).argtypes = args
            getattr(H, nm).restype = i
        _hip = H
    return _hip


def _hipcheck(rc, what):
    if rc != 0:
        raise TskError(-8, f"{what} failed with hipError {rc}")


class DeviceArray:
    """A device buffer (or a strided view of one) of dtype f32/f16/bf16/i32/u8.
    shape/strides are numpy-style (strides in elements), C-contiguous by default."""

    def __init__(self, shape, dtype="f32", _base=None, _ptr=None, _strides=None):
        self.shape = tuple(int(x) for x in shape)
        self.dtype = dtype
        self.ttype, self.itemsize, self.npdtype = DTYPES[dtype]
        if _strides is None:
            st, acc = [], 1
            for d in reversed(self.shape):
                st.append(acc)
                acc *= d
            _strides = tuple(reversed(st))
        self.strides = tuple(int(x) for x in _strides)
        self._base = _base
        if _ptr is not None:
            self.ptr = _ptr
        else:
            n = 1
            for d in self.shape:
                n *= d
            p = ctypes.c_void_p()
            _hipcheck(hip().hipMalloc(ctypes.byref(p), max(n * self.itemsize, 256)), "hipMalloc")
            self.ptr = p.value
            self._owner = True

    def __del__(self):
        if getattr(self, "_owner", False) and self.ptr:
            try:
                hip().hipFree(ctypes.c_void_p(self.ptr))
            except Exception:
                pass
            self.ptr = None

    # accessors used by desc()
    def stride(self, dim=None):
        return self.strides if dim is None else self.strides[dim]

    def element_size(self):
        return self.itemsize

    def data_ptr(self):
        return self.ptr

    @property
    def nbytes(self):
        n = 1
        for d in self.shape:
            n *= d
        return n * self.itemsize

    def contiguous(self):
        exp = DeviceArray(self.shape, self.dtype, _ptr=0).strides
        return self.strides == exp

    @staticmethod
    def from_numpy(a, dtype=None):
        import numpy as np
        if dtype is None:
            dtype = {np.dtype("float32"): "f32", np.dtype("float16"): "f16", np.dtype("int32"): "i32",
                     np.dtype("uint8"): "u8"}[a.dtype]
        a = np.ascontiguousarray(a)
        d = DeviceArray(a.shape, dtype)
        _hipcheck(hip().hipMemcpy(ctypes.c_void_p(d.ptr), ctypes.c_void_p(a.ctypes.data), a.nbytes, 1),
                  "hipMemcpy H2D")
        return d

    def numpy(self):
        import numpy as np
        if not self.contiguous():
            raise ValueError("numpy() needs a contiguous array")
        out = np.empty(self.shape, dtype=self.npdtype)
        synchronize()
        _hipcheck(hip().hipMemcpy(ctypes.c_void_p(out.ctypes.data), ctypes.c_void_p(self.ptr), out.nbytes, 2),
                  "hipMemcpy D2H")
        return out

    def view(self, offset, shape, strides):
        """strided view starting `offset` elements into this buffer"""
        return DeviceArray(shape, self.dtype, _base=self, _ptr=self.ptr + offset * self.itemsize,
                           _strides=strides)

    def select(self, dim, index):
        """view with dimension `dim` fixed at `index` (like a[:, index] for dim 1)"""
        off = index * self.strides[dim]
        shape = self.shape[:dim] + self.shape[dim + 1:]
        strides = self.strides[:dim] + self.strides[dim + 1:]
        return self.view(off, shape, strides)


def synchronize():
    _hipcheck(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        _hipcheck(hip().hipEventCreate(ctypes.byref(p)), "hipEventCreate")
        self.h = p

    def record(self, stream=None):
        _hipcheck(hip().hipEventRecord(self.h, _stream(stream)), "hipEventRecord")

    def elapsed_ms(self, end):
        _hipcheck(hip().hipEventSynchronize(end.h), "hipEventSynchronize")
        ms = ctypes.c_float()
        _hipcheck(hip().hipEventElapsedTime(ctypes.byref(ms), self.h, end.h), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            hip().hipEventDestroy(self.h)
        except Exception:
            pass


def empty(shape, dtype="f32"):
    return DeviceArray(shape, dtype)


def to_device(a, dtype=None):
    return DeviceArray.from_numpy(a, dtype)


def bf16_to_device(bits):
    """uint16 numpy array of bf16 bit patterns -> bf16 DeviceArray"""
    import numpy as np
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    d = DeviceArray(bits.shape, "bf16")
    _hipcheck(hip().hipMemcpy(ctypes.c_void_p(d.ptr), ctypes.c_void_p(bits.ctypes.data), bits.nbytes, 1),
              "hipMemcpy H2D")
    return d


# ---------------------------------------------------------------- descriptors
def desc(t, ttype=None):
    """tsk_tensor view of a DeviceArray: ne = reversed shape, nb = reversed byte strides.
    A Q8_0 tensor is a u8 array of shape (rows, K/32, 34)."""
    d = TskTensor()
    ttype = t.ttype if ttype is None else ttype
    d.type = ttype
    if ttype == Q8_0:
        rows, nblk = t.shape[0], t.shape[1]
        ne = [nblk * 32, rows]
        nb = [34, t.stride(0)]
    elif ttype == Q8_0_SPLIT:
        ne = list(t.logical_shape)
        nb = [1, ne[0]]
    else:
        es = t.element_size()
        ne = list(t.shape)[::-1]
        nb = [s * es for s in t.stride()][::-1]
    while len(ne) < 4:
        nb.append(nb[-1] * ne[-1] if ne else 4)
        ne.append(1)
    for k in range(4):
        d.ne[k] = int(ne[k])
        d.nb[k] = int(nb[k])
    d.data = t.data_ptr()
    return d


class Stream:
    """A HIP stream of the runtime libtsk.so links (default priority)."""

    def __init__(self):
        p = ctypes.c_void_p()
        _hipcheck(hip().hipStreamCreate(ctypes.byref(p)), "hipStreamCreate")
        self.h = p

    def synchronize(self):
        _hipcheck(hip().hipStreamSynchronize(self.h), "hipStreamSynchronize")

    def destroy(self):
        if getattr(self, "h", None) is not None:
            release_workspace(self)
            hip().hipStreamDestroy(self.h)
            self.h = None


class Graph:
    """The work a function enqueues on `stream`, captured into a HIP graph
    (hipStreamCaptureModeGlobal: a call that is not allowed under capture,
    hipMalloc among them, fails the capture) and replayed with launch()."""

    def __init__(self, stream, fn):
        H = hip()
        _hipcheck(H.hipStreamBeginCapture(stream.h, 0), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            g = ctypes.c_void_p()
            rc = H.hipStreamEndCapture(stream.h, ctypes.byref(g))
        _hipcheck(rc, "hipStreamEndCapture")
        self.graph = g
        e = ctypes.c_void_p()
        _hipcheck(H.hipGraphInstantiate(ctypes.byref(e), g, None, None, 0), "hipGraphInstantiate")
        self.exec = e
        self.stream = stream

    def launch(self):
        _hipcheck(hip().hipGraphLaunch(self.exec, self.stream.h), "hipGraphLaunch")

    def destroy(self):
        if getattr(self, "exec", None) is not None:
            hip().hipGraphExecDestroy(self.exec)
            hip().hipGraphDestroy(self.graph)
            self.exec = None


def _stream(stream=None):
    """hipStream_t of a Stream (None: the null stream)."""
    return None if stream is None else stream.h


def _ref(x):
    return ctypes.byref(x) if x is not None else None


# ---------------------------------------------------------------- operators
def mul_mat(a, b, bias=None, out=None, a_type=None, out_dtype="f32", stream=None):
    """ggml_mul_mat(a, b) (+bias): a (M, K) weights, b (..., N, K) -> (..., N, M)."""
    init()
    at = a_type if a_type is not None else a.ttype
    M = a.shape[0] if at != Q8_0_SPLIT else a.logical_shape[1]
    if out is None:
        out = DeviceArray(tuple(b.shape[:-1]) + (M,), out_dtype)
    da, db, dd = desc(a, at), desc(b), desc(out)
    dbias = desc(bias) if bias is not None else None
    check(load().tsk_mul_mat(ctypes.byref(da), ctypes.byref(db), _ref(dbias), ctypes.byref(dd),
                             _stream(stream)))
    return out


def mul_mat_noalloc(a, b, bias=None, out=None, a_type=None, out_dtype="f32", stream=None):
    """mul_mat through tsk_mul_mat_noalloc (scratch in the library's fixed per-GPU array)."""
    init()
    at = a_type if a_type is not None else a.ttype
    M = a.shape[0] if at != Q8_0_SPLIT else a.logical_shape[1]
    if out is None:
        out = DeviceArray(tuple(b.shape[:-1]) + (M,), out_dtype)
    da, db, dd = desc(a, at), desc(b), desc(out)
    dbias = desc(bias) if bias is not None else None
    check(load().tsk_mul_mat_noalloc(ctypes.byref(da), ctypes.byref(db), _ref(dbias), ctypes.byref(dd),
                                     _stream(stream)))
    return out


def flash_attn_ext(q, k, v, mask=None, scale=0.125, max_bias=0.0, softcap=0.0, prec=PREC_F32,
                   out=None, out_dtype="f32", stream=None):
    """q (B, H, Nq, D), k/v (B, Hkv, Nkv, D) -> (B, Nq, H, D) (ggml's permuted result)."""
    init()
    B, H, Nq, D = q.shape
    if out is None:
        out = DeviceArray((B, Nq, H, v.shape[-1]), out_dtype)
    dq, dk, dv, dd = desc(q), desc(k), desc(v), desc(out)
    dm = desc(mask) if mask is not None else None
    check(load().tsk_flash_attn_ext(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv), _ref(dm),
                                    scale, max_bias, softcap, prec, ctypes.byref(dd), _stream(stream)))
    return out


def t5_attention(q, k, v, rel_lut, key_valid, scale=1.0, out=None):
    """T5 self-attention with a relative-position bias table: q/k/v (1, H, n, 64)
    views, rel_lut (H, 2 n_max - 1) f32, key_valid u8 (n,) -> (1, n, H, 64)."""
    init()
    _, H, n, D = q.shape
    if out is None:
        out = DeviceArray((1, n, H, D), "f32")
    dq, dk, dv, dl, dd = desc(q), desc(k), desc(v), desc(rel_lut), desc(out)
    check(load().tsk_t5_attention(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv), ctypes.byref(dl),
                                  ctypes.c_void_p(key_valid.data_ptr()), scale, ctypes.byref(dd), _stream()))
    return out


def workspace_size(op, srcs, dst):
    """tsk_workspace_size: srcs are DeviceArrays, (DeviceArray, ttype) pairs or None."""
    P = ctypes.POINTER(TskTensor)
    descs = []
    for x in srcs:
        if x is None:
            descs.append(None)
        elif isinstance(x, tuple):
            descs.append(desc(x[0], x[1]))
        else:
            descs.append(desc(x))
    arr = (P * len(descs))(*[ctypes.pointer(d) if d is not None else P() for d in descs])
    dd = desc(dst)
    n = ctypes.c_size_t()
    check(load().tsk_workspace_size(op, arr, len(descs), ctypes.byref(dd), ctypes.byref(n)))
    return n.value


def set_workspace(buf, stream=None):
    """Bind DeviceArray buf (or None to unbind) as the workspace of `stream`."""
    init()
    if buf is None:
        check(load().tsk_set_workspace(_stream(stream), None, 0))
    else:
        check(load().tsk_set_workspace(_stream(stream), ctypes.c_void_p(buf.data_ptr()), buf.nbytes))


def release_workspace(stream=None):
    init()
    check(load().tsk_release_workspace(_stream(stream)))


def rms_norm_mul(x, w, eps, out=None):
    init()
    out = DeviceArray(x.shape, x.dtype) if out is None else out
    dx, dd = desc(x), desc(out)
    dw = desc(w) if w is not None else None
    check(load().tsk_rms_norm_mul(ctypes.byref(dx), _ref(dw), eps, ctypes.byref(dd), _stream()))
    return out


def norm(x, eps, out=None):
    init()
    out = DeviceArray(x.shape, x.dtype) if out is None else out
    dx, dd = desc(x), desc(out)
    check(load().tsk_norm(ctypes.byref(dx), eps, ctypes.byref(dd), _stream()))
    return out


def rope_ext(x, pos, n_dims, freq_base=10000.0, freq_scale=1.0, mode=ROPE_NORMAL, out=None):
    """x (B, S, H, D) i.e. ggml [D, H, S, B]; pos int32 (S,)."""
    init()
    out = DeviceArray(x.shape, x.dtype) if out is None else out
    dx, dp, dd = desc(x), desc(pos), desc(out)
    check(load().tsk_rope_ext(ctypes.byref(dx), ctypes.byref(dp), n_dims, mode, freq_base, freq_scale,
                              0.0, 1.0, ctypes.byref(dd), _stream()))
    return out


def qk_norm_rope(x, w, pos, eps=1e-6, n_dims=64, freq_base=10000.0, freq_scale=1.0, out=None):
    init()
    out = DeviceArray(x.shape, x.dtype) if out is None else out
    dx, dw, dd = desc(x), desc(w), desc(out)
    dp = desc(pos) if pos is not None else None
    check(load().tsk_qk_norm_rope(ctypes.byref(dx), ctypes.byref(dw), _ref(dp), eps, n_dims, freq_base,
                                  freq_scale, ctypes.byref(dd), _stream()))
    return out


def rms_norm_q8_0(x, w, eps):
    """T5's rms_norm * w straight into ggml Q8_0 blocks: x (rows, n) f32 -> u8 (rows, n/32, 34)."""
    init()
    rows, n = x.shape
    out = DeviceArray((rows, n // 32, 34), "u8")
    dx, dw, dd = desc(x), desc(w), desc(out, Q8_0)
    check(load().tsk_rms_norm_q8_0(ctypes.byref(dx), ctypes.byref(dw), eps, ctypes.byref(dd), _stream()))
    return out


def q8_0_quantize(x):
    """(rows, K) f32 -> (rows, K/32, 34) u8 ggml block_q8_0 bytes."""
    init()
    rows, K = x.shape
    out = DeviceArray((rows, K // 32, 34), "u8")
    dx, dd = desc(x), desc(out, Q8_0)
    check(load().tsk_q8_0_quantize(ctypes.byref(dx), ctypes.byref(dd), _stream()))
    return out


class SplitQ8:
    """Q8_0 weights repacked into int8 / fp16 planes (TSK_TYPE_Q8_0_SPLIT)."""

    def __init__(self, buf, K, M):
        self.buf, self.logical_shape = buf, (K, M)

    def data_ptr(self):
        return self.buf.data_ptr()


def q8_0_repack(blocks):
    init()
    rows, nb = blocks.shape[0], blocks.shape[1]
    K = nb * 32
    buf = DeviceArray((load().tsk_q8_0_split_nbytes(K, rows),), "u8")
    sp = SplitQ8(buf, K, rows)
    ds, dd = desc(blocks, Q8_0), desc(sp, Q8_0_SPLIT)
    check(load().tsk_q8_0_repack(ctypes.byref(ds), ctypes.byref(dd), _stream()))
    return sp


def q8_0_dequantize(x):
    init()
    if isinstance(x, SplitQ8):
        K, rows = x.logical_shape
        dx = desc(x, Q8_0_SPLIT)
    else:
        rows, K = x.shape[0], x.shape[1] * 32
        dx = desc(x, Q8_0)
    out = DeviceArray((rows, K), "f32")
    dd = desc(out)
    check(load().tsk_q8_0_dequantize(ctypes.byref(dx), ctypes.byref(dd), _stream()))
    return out


# ---------------------------------------------------------------- convolution / SwiGLU
def conv_len(iw, kw, s0=1, p0=1, d0=1):
    return (iw + 2 * p0 - d0 * (kw - 1) - 1) // s0 + 1


def im2col_1d(kernel_shape, x, s0=1, p0=1, d0=1, out_dtype="f32"):
    """ggml_im2col 1-D: kernel_shape (OC, IC, KW); x (N, IC, IW) f32 (any
    strides, e.g. a transposed view) -> (N, OW, IC*KW)."""
    init()
    OC, IC, KW = kernel_shape
    N, _, IW = x.shape
    out = DeviceArray((N, conv_len(IW, KW, s0, p0, d0), IC * KW), out_dtype)
    k = TskTensor()
    k.type = F32
    k.ne[0], k.ne[1], k.ne[2], k.ne[3] = KW, IC, OC, 1
    dx, dd = desc(x), desc(out)
    check(load().tsk_im2col_1d(ctypes.byref(k), ctypes.byref(dx), s0, p0, d0, ctypes.byref(dd), _stream()))
    return out


def conv1d_pack_weight(w):
    """(OC, IC, KW) kernel (ggml ne [KW, IC, OC]) -> a copy laid out kw-major,
    returned as an (OC, IC, KW) view with element strides (KW*IC, 1, IC)."""
    init()
    OC, IC, KW = w.shape
    buf = DeviceArray((OC * KW * IC,), w.dtype)
    out = buf.view(0, (OC, IC, KW), (KW * IC, 1, IC))
    dw, dd = desc(w), desc(out)
    check(load().tsk_conv1d_pack_weight(ctypes.byref(dw), ctypes.byref(dd), _stream()))
    return out


def conv1d(w, x, bias=None, s0=1, p0=1, d0=1, out=None, out_dtype="f32"):
    """conv_cl: w (OC, IC, KW) kernel, x (B, IW, IC) channels fastest -> (B, OW, OC)."""
    init()
    OC, IC, KW = w.shape
    B, IW, _ = x.shape
    if out is None:
        out = DeviceArray((B, conv_len(IW, KW, s0, p0, d0), OC), out_dtype)
    dw, dx, dd = desc(w), desc(x), desc(out)
    db = desc(bias) if bias is not None else None
    check(load().tsk_conv1d(ctypes.byref(dw), _ref(db), ctypes.byref(dx), s0, p0, d0, ctypes.byref(dd), _stream()))
    return out


def swiglu(a, b, out=None):
    """ggml_mul(ggml_silu(a), b), f32."""
    init()
    out = DeviceArray(a.shape, "f32") if out is None else out
    da, db, dd = desc(a), desc(b), desc(out)
    check(load().tsk_swiglu(ctypes.byref(da), ctypes.byref(db), ctypes.byref(dd), _stream()))
    return out


def conv_mlp_swiglu(w1, w3, w2, x, out=None, out_dtype="f32"):
    """convmlp: kernels (HID, IC, KW), (HID, IC, KW), (OC, HID, KW); x (B, IW, IC) -> (B, OW, OC)."""
    init()
    B, IW, _ = x.shape
    if out is None:
        ow = conv_len(conv_len(IW, w1.shape[2]), w2.shape[2])
        out = DeviceArray((B, ow, w2.shape[0]), out_dtype)
    d1, d3, d2, dx, dd = desc(w1), desc(w3), desc(w2), desc(x), desc(out)
    check(load().tsk_conv_mlp_swiglu(ctypes.byref(d1), ctypes.byref(d3), ctypes.byref(d2), ctypes.byref(dx),
                                     ctypes.byref(dd), _stream()))
    return out


def mlp_swiglu(w1, w3, w2, x, out=None, out_dtype="f32"):
    """mlp: weights (HID, IC), (HID, IC), (OC, HID); x (..., IC) -> (..., OC)."""
    init()
    if out is None:
        out = DeviceArray(tuple(x.shape[:-1]) + (w2.shape[0],), out_dtype)
    d1, d3, d2, dx, dd = desc(w1), desc(w3), desc(w2), desc(x), desc(out)
    check(load().tsk_mlp_swiglu(ctypes.byref(d1), ctypes.byref(d3), ctypes.byref(d2), ctypes.byref(dx),
                                ctypes.byref(dd), _stream()))
    return out


# ---------------------------------------------------------------- MM-DiT driver
def synthetic_weights(tensors, seed=1234, std=0.02):
    """Seeded random-init weights {name: float32 array of shape (ne1, ne0)}.
    Matrices (ne1 > 1) are N(0, std) rounded to bf16 (RNE) so every consumer
    sees the values the device holds; biases are N(0, std); RMSNorm weights
    are 1 + N(0, std). Each tensor has its own stream (seed, crc32(name))."""
    import zlib

    import numpy as np
    out = {}
    for name, ne in tensors:
        rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
        n = int(ne[0]) * int(ne[1])
        w = rng.standard_normal(n, dtype=np.float32) * np.float32(std)
        if name.endswith("norm.weight"):
            w += np.float32(1.0)
        if ne[1] > 1:
            u = w.view(np.uint32)
            u = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
            w = u.view(np.float32)
        out[name] = w.reshape(int(ne[1]), int(ne[0])) if ne[1] > 1 else w
    return out


def dit_config(**kw):
    c = DitConfig()
    load().tsk_dit_default_config(ctypes.byref(c))
    for k_, v_ in kw.items():
        setattr(c, k_, v_)
    return c


class Dit:
    """ts_dit counterpart: named BF16 weights on the GPU, forward() and sample()."""

    def __init__(self, cfg=None):
        init()
        self.cfg = cfg if cfg is not None else dit_config()
        h = ctypes.c_void_p()
        check(load().tsk_dit_create(ctypes.byref(self.cfg), ctypes.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            load().tsk_dit_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        """[(name, ggml ne tuple)] of every weight the driver expects."""
        L = load()
        out = []
        for k_ in range(L.tsk_dit_n_tensors(self.h)):
            nm = ctypes.c_char_p()
            ne = (ctypes.c_int64 * 4)()
            check(L.tsk_dit_tensor_info(self.h, k_, ctypes.byref(nm), ne))
            out.append((nm.value.decode(), tuple(ne)))
        return out

    def set_tensor(self, name, host_f32):
        """host_f32: contiguous numpy float32 array."""
        host_f32 = np.ascontiguousarray(host_f32, dtype=np.float32)
        check(load().tsk_dit_set_tensor(self.h, name.encode(), host_f32.ctypes.data, host_f32.size))

    def set_tensor_q8_0(self, name, blocks):
        """ggml Q8_0 blocks (uint8, 34 bytes per 32 values) of a Q8_0 block projection."""
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        check(load().tsk_dit_set_tensor_q8_0(self.h, name.encode(), blocks.ctypes.data, blocks.nbytes))

    def tensor_types(self):
        """{name: stored type id} (BF16 / Q8_0 / F32)"""
        L = load()
        return {nm: L.tsk_dit_tensor_type(self.h, k_) for k_, (nm, _) in enumerate(self.tensors())}

    def forward(self, latent, t, text):
        """ts_dit::forward layouts, host numpy arrays: latent (B, L, T) (ggml ne =
        [T, L, B]), t (B,), text (B, text_seq, hidden) -> flow (B, T, L)."""
        import numpy as np
        latent = np.ascontiguousarray(latent, dtype=np.float32)
        t = np.ascontiguousarray(t, dtype=np.float32)
        text = np.ascontiguousarray(text, dtype=np.float32)
        B, L, T = latent.shape
        flow = np.empty((B, T, L), np.float32)
        check(load().tsk_dit_forward(self.h, B, T, latent.ctypes.data, t.ctypes.data, text.ctypes.data,
                                     flow.ctypes.data, _stream()))
        return flow

    def forward_device(self, latent, t, text, flow):
        """DeviceArrays latent (B, L, T), text (B, S, H), flow out (B, T, L) f32; t host numpy (B,)."""
        import numpy as np
        t = np.ascontiguousarray(t, dtype=np.float32)
        B, _, T = latent.shape
        check(load().tsk_dit_forward_device(self.h, B, T, ctypes.c_void_p(latent.data_ptr()),
                                            t.ctypes.data, ctypes.c_void_p(text.data_ptr()),
                                            ctypes.c_void_p(flow.data_ptr()), _stream()))
        return flow

    ROLES = ("qkv", "out", "fc1", "fc2", "attn", "adaln", "other")

    def timing(self, enable=True):
        check(load().tsk_dit_timing(self.h, int(bool(enable))))

    def timing_read(self):
        """{role: (ms_total, launches, flop, bytes)} since the last timing(True)."""
        out = {}
        for r, nm in enumerate(self.ROLES):
            ms, n, fl, by = ctypes.c_double(), ctypes.c_int64(), ctypes.c_double(), ctypes.c_double()
            check(load().tsk_dit_timing_read(self.h, r, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(fl),
                                             ctypes.byref(by)))
            out[nm] = (ms.value, n.value, fl.value, by.value)
        return out

    def sample(self, noise, text_cond, text_uncond, steps=24, cfg_scale=5.0):
        """ts_dit::sample layouts: noise (L, T) (ggml ne = [T, L]), text (text_seq, hidden)
        -> (latent (L, T), flow0 (L, T))."""
        import numpy as np
        noise = np.ascontiguousarray(noise, dtype=np.float32)
        text_cond = np.ascontiguousarray(text_cond, dtype=np.float32)
        text_uncond = np.ascontiguousarray(text_uncond, dtype=np.float32)
        L, T = noise.shape
        out = np.empty_like(noise)
        flow0 = np.empty_like(noise)
        check(load().tsk_dit_sample(self.h, T, noise.ctypes.data, text_cond.ctypes.data,
                                    text_uncond.ctypes.data, steps, cfg_scale, out.ctypes.data,
                                    flow0.ctypes.data, _stream()))
        return out, flow0


# ---------------------------------------------------------------- the reference's MM-DiT graph
def mmdit_config(**kw):
    c = MMDitConfig()
    load().tsk_mmdit_default_config(ctypes.byref(c))
    for k_, v_ in kw.items():
        setattr(c, k_, v_)
    return c


def mmdit_synthetic_weights(tensors, seed=1234, std=0.02):
    """Seeded random-init weights {name: float32 array in ggml / PyTorch order}
    for [(name, ne, type)]: BF16 tensors N(0, std) rounded to bf16 (RNE), F32
    matrices and biases N(0, std), q/k norm weights 1 + N(0, std), the learned
    empty features N(0, 1). Each tensor has its own stream (seed, crc32(name))."""
    import zlib
    out = {}
    for name, ne, ty in tensors:
        rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
        shape = tuple(int(x) for x in reversed(ne))
        while len(shape) > 1 and shape[0] == 1:
            shape = shape[1:]
        n = int(np.prod(shape))
        sd = 1.0 if name.startswith("empty_") else std
        w = rng.standard_normal(n, dtype=np.float32) * np.float32(sd)
        if name.endswith("norm.weight"):
            w += np.float32(1.0)
        if ty == BF16:
            u = w.view(np.uint32)
            u = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
            w = u.view(np.float32)
        out[name] = w.reshape(shape)
    return out


def mmdit_pool_weights(tensors, seed=1234, std=0.02, pool_size=1 << 24):
    """(name, array) pairs of random-init weights for the reference graph's
    1.28 G parameters, generated lazily: every matrix a window (at a seeded
    offset, wrapping) of one pool of N(0, std) values rounded to bf16; vectors
    N(0, std) (q/k norm weights 1 + N(0, std)); the learned empties N(0, 1).
    Drawing 1.28 G fresh normals takes minutes on a host; the windows give
    every matrix its own values at the cost of shared statistics."""
    def window(pool, off, n):
        w = np.empty(n, np.float32)
        i = 0
        while i < n:
            k = min(n - i, pool.size - off)
            w[i:i + k] = pool[off:off + k]
            i, off = i + k, 0
        return w
    rng = np.random.default_rng(seed)
    pool = (rng.standard_normal(pool_size, dtype=np.float32) * np.float32(std)).view(np.uint32)
    pool = ((pool + np.uint32(0x7FFF) + ((pool >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000))
    pool = pool.view(np.float32)
    for name, ne, _ty in tensors:
        shape = tuple(int(x) for x in reversed(ne))
        while len(shape) > 1 and shape[0] == 1:
            shape = shape[1:]
        n = int(np.prod(shape))
        if name.startswith("empty_"):
            w = rng.standard_normal(n, dtype=np.float32)
        elif len(shape) == 1:
            w = rng.standard_normal(n, dtype=np.float32) * np.float32(std)
            if name.endswith("norm.weight"):
                w += np.float32(1.0)
        else:
            w = window(pool, int(rng.integers(0, pool.size)), n)
        yield name, w.reshape(shape)


class MMDit:
    """ts_dit counterpart running the reference's graph (src/mmdit.cpp:119-376):
    named BF16 / F32 / Q8_0 weights on the GPU, forward() and sample()."""

    def __init__(self, cfg=None, gguf=None):
        """cfg: sizes, capacities and weight_type; gguf: a Gguf file whose
        tensors' types the model takes and whose weights it loads
        (ts_dit::load)"""
        init()
        self.cfg = cfg if cfg is not None else mmdit_config()
        h = ctypes.c_void_p()
        if gguf is None:
            check(load().tsk_mmdit_create(ctypes.byref(self.cfg), ctypes.byref(h)))
        else:
            check(load().tsk_mmdit_create_from_gguf(gguf.h, ctypes.byref(self.cfg), ctypes.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            load().tsk_mmdit_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        """[(name, ggml ne (3), type id)] of every weight"""
        L = load()
        out = []
        for k_ in range(L.tsk_mmdit_n_tensors(self.h)):
            nm = ctypes.c_char_p()
            ne = (ctypes.c_int64 * 4)()
            check(L.tsk_mmdit_tensor_info(self.h, k_, ctypes.byref(nm), ne))
            out.append((nm.value.decode(), tuple(ne)[:3], L.tsk_mmdit_tensor_type(self.h, k_)))
        return out

    def set_tensor(self, name, host_f32):
        host_f32 = np.ascontiguousarray(host_f32, dtype=np.float32)
        check(load().tsk_mmdit_set_tensor(self.h, name.encode(), host_f32.ctypes.data, host_f32.size))

    def set_tensor_q8_0(self, name, blocks):
        """Q8_0 blocks (bytes / uint8 array) of a tensor held as Q8_0"""
        b = np.ascontiguousarray(np.frombuffer(bytes(blocks), np.uint8))
        check(load().tsk_mmdit_set_tensor_q8_0(self.h, name.encode(), b.ctypes.data, b.size))

    def load_gguf(self, gguf):
        check(load().tsk_mmdit_load_gguf(self.h, gguf.h))

    @staticmethod
    def _c(a):
        return np.ascontiguousarray(a, dtype=np.float32)

    def forward(self, latent, t, clip, sync, text, t5, g):
        """ts_dit::forward layouts with the batch outermost: latent (B, L, T),
        t (B,), clip (B, S_c, clip_dim), sync (B, S_s, sync_dim), text
        (B, text_seq, clip_dim), t5 (B, text_seq, t5_dim), g (B, clip_dim)
        -> flow (B, T, L)"""
        latent, t, clip, sync, text, t5, g = (self._c(a) for a in (latent, t, clip, sync, text, t5, g))
        B, L, T = latent.shape
        flow = np.empty((B, T, L), np.float32)
        check(load().tsk_mmdit_forward(self.h, B, T, latent.ctypes.data, t.ctypes.data, clip.shape[1],
                                       clip.ctypes.data, sync.shape[1], sync.ctypes.data, text.ctypes.data,
                                       t5.ctypes.data, g.ctypes.data, flow.ctypes.data, _stream()))
        return flow

    def forward_device(self, latent, t, clip, sync, text, t5, g, flow):
        """DeviceArrays in forward()'s layouts, flow out (B, T, L); t host (B,)"""
        t = np.ascontiguousarray(t, dtype=np.float32)
        B, _, T = latent.shape
        d = lambda a: ctypes.c_void_p(a.data_ptr())
        check(load().tsk_mmdit_forward_device(self.h, B, T, d(latent), t.ctypes.data, clip.shape[1], d(clip),
                                              sync.shape[1], d(sync), d(text), d(t5), d(g), d(flow), _stream()))
        return flow

    def debug(self, enable=True):
        """keep the stage outputs of every forward (src/mmdit.cpp:333-336)"""
        check(load().tsk_mmdit_debug(self.h, int(bool(enable))))

    def stage(self, name):
        """a stage output of the last forward, flat in [B][S][H] order"""
        L = load()
        n = L.tsk_mmdit_debug_size(self.h, name.encode())
        check(int(n) if n < 0 else 0)
        out = np.empty(int(n), np.float32)
        check(L.tsk_mmdit_debug_get(self.h, name.encode(), out.ctypes.data, n))
        return out

    def sample(self, noise, clip, sync, text, t5, g, steps=24, cfg_scale=5.0):
        """ts_dit::sample layouts: noise (L, T), clip (S_c, clip_dim), sync
        (S_s, sync_dim), text (text_seq, clip_dim), t5 (text_seq, t5_dim), g
        (clip_dim,) -> (latent (L, T), flow0 (L, T))"""
        noise, clip, sync, text, t5, g = (self._c(a) for a in (noise, clip, sync, text, t5, g))
        L, T = noise.shape
        out = np.empty_like(noise)
        flow0 = np.empty_like(noise)
        check(load().tsk_mmdit_sample(self.h, T, noise.ctypes.data, clip.shape[0], clip.ctypes.data, sync.shape[0],
                                      sync.ctypes.data, text.ctypes.data, t5.ctypes.data, g.ctypes.data, steps,
                                      cfg_scale, out.ctypes.data, flow0.ctypes.data, _stream()))
        return out, flow0


# ---------------------------------------------------------------- Oobleck VAE decoder (ts_vae)
def vae_config(**kw):
    c = VaeConfig()
    load().tsk_vae_default_config(ctypes.byref(c))
    if "c_mults" in kw:
        c.c_mults[:] = kw.pop("c_mults")
    if "strides" in kw:
        c.strides[:] = kw.pop("strides")
    for k_, v_ in kw.items():
        setattr(c, k_, v_)
    return c


def vae_synthetic_weights(tensors, seed=77, snake_std=0.5):
    """seeded weights {name: float32 array in ggml / PyTorch order}: conv
    kernels N(0, 1 / (K IC)) (variance-preserving), biases N(0, 0.02), snake
    alpha / beta N(0, snake_std) (log-scale parameters)"""
    import zlib
    out = {}
    for name, ne in tensors:
        rng = np.random.default_rng([seed, zlib.crc32(name.encode())])
        shape = tuple(int(x) for x in reversed(ne))
        while len(shape) > 1 and shape[0] == 1:
            shape = shape[1:]
        n = int(np.prod(shape))
        if name.endswith(".weight"):
            w = rng.standard_normal(n) / np.sqrt(ne[0] * ne[1])
        elif name.endswith(".bias"):
            w = rng.standard_normal(n) * 0.02
        else:
            w = rng.standard_normal(n) * snake_std
        out[name] = w.astype(np.float32).reshape(shape)
    return out


class Vae:
    """ts_vae counterpart (src/vae_decoder.h:6-17): named F32 weights on the
    GPU and decode()"""

    def __init__(self, cfg=None):
        init()
        self.cfg = cfg if cfg is not None else vae_config()
        h = ctypes.c_void_p()
        check(load().tsk_vae_create(ctypes.byref(self.cfg), ctypes.byref(h)))
        self.h = h
        self.hop = load().tsk_vae_hop(self.h)

    def close(self):
        if getattr(self, "h", None):
            load().tsk_vae_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        L = load()
        out = []
        for k_ in range(L.tsk_vae_n_tensors(self.h)):
            nm = ctypes.c_char_p()
            ne = (ctypes.c_int64 * 4)()
            check(L.tsk_vae_tensor_info(self.h, k_, ctypes.byref(nm), ne))
            out.append((nm.value.decode(), tuple(ne)[:3]))
        return out

    def set_tensor(self, name, host_f32):
        host_f32 = np.ascontiguousarray(host_f32, dtype=np.float32)
        check(load().tsk_vae_set_tensor(self.h, name.encode(), host_f32.ctypes.data, host_f32.size))

    def decode(self, latent):
        """latent (latent_dim, T) (ggml ne = [T, latent_dim]) -> audio (out_channels, T * hop)"""
        latent = np.ascontiguousarray(latent, dtype=np.float32)
        L, T = latent.shape
        audio = np.empty((self.cfg.out_channels, T * self.hop), np.float32)
        ta = ctypes.c_int64()
        check(load().tsk_vae_decode(self.h, T, latent.ctypes.data, audio.ctypes.data, ctypes.byref(ta), _stream()))
        assert ta.value == T * self.hop
        return audio

    def decode_device(self, latent, audio):
        """DeviceArrays latent (latent_dim, T), audio out (out_channels, T * hop)"""
        check(load().tsk_vae_decode_device(self.h, latent.shape[1], ctypes.c_void_p(latent.data_ptr()),
                                           ctypes.c_void_p(audio.data_ptr()), _stream()))
        return audio


# ---------------------------------------------------------------- T5 encoder (ts_t5)
def t5_config(**kw):
    c = T5Config()
    load().tsk_t5_default_config(ctypes.byref(c))
    for k_, v_ in kw.items():
        setattr(c, k_, v_)
    return c


class T5:
    """ts_t5 counterpart (src/t5_encoder.cpp:28-104): named Q8_0 / F32 weights on
    the GPU and the encoder layers on embedded tokens."""

    def __init__(self, cfg=None):
        init()
        self.cfg = cfg if cfg is not None else t5_config()
        h = ctypes.c_void_p()
        check(load().tsk_t5_create(ctypes.byref(self.cfg), ctypes.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            load().tsk_t5_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        """[(name, ggml ne tuple, type)]"""
        L = load()
        out = []
        for k_ in range(L.tsk_t5_n_tensors(self.h)):
            nm, ne, ty = ctypes.c_char_p(), (ctypes.c_int64 * 4)(), ctypes.c_int()
            check(L.tsk_t5_tensor_info(self.h, k_, ctypes.byref(nm), ne, ctypes.byref(ty)))
            out.append((nm.value.decode(), tuple(ne), ty.value))
        return out

    def set_tensor(self, name, data):
        """data: numpy Q8_0 blocks (uint8, 34 bytes per 32 values) or float32."""
        import numpy as np
        data = np.ascontiguousarray(data)
        check(load().tsk_t5_set_tensor(self.h, name.encode(), data.ctypes.data, data.nbytes))

    def encode(self, x, ids, layers=None, final_norm=True):
        """x (n, d_model) float32 embedded tokens, ids (n,) int32 (0 = padded key) -> (n, d_model);
        layers = (begin, end) runs only those layers (default: all)."""
        import numpy as np
        x = np.ascontiguousarray(x, dtype=np.float32)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty_like(x)
        b, e = layers if layers is not None else (0, self.cfg.n_layers)
        check(load().tsk_t5_encode_range(self.h, x.shape[0], x.ctypes.data, ids.ctypes.data, b, e,
                                         int(final_norm), out.ctypes.data, _stream()))
        return out

    def encode_device(self, x, ids, out=None):
        """x: (n, d_model) f32 DeviceArray, ids: (n,) int32 host array -> (n, d_model) DeviceArray."""
        import numpy as np
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = DeviceArray(x.shape, "f32") if out is None else out
        check(load().tsk_t5_encode_device(self.h, x.shape[0], x.data_ptr(), ids.ctypes.data, out.data_ptr(),
                                          _stream()))
        return out


# ---------------------------------------------------------------- GGUF files
class Gguf:
    """A GGUF file opened by the library's reader (host only; no GPU needed)."""

    TYPES = {0: "f32", 1: "f16", 8: "q8_0", 30: "bf16"}

    def __init__(self, path):
        h = ctypes.c_void_p()
        check(load().tsk_gguf_open(str(path).encode(), ctypes.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            load().tsk_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        """[(name, ggml ne tuple, ggml type)]"""
        out = []
        for k_ in range(load().tsk_gguf_n_tensors(self.h)):
            nm, ne, ty = ctypes.c_char_p(), (ctypes.c_int64 * 4)(), ctypes.c_int()
            check(load().tsk_gguf_tensor_info(self.h, k_, ctypes.byref(nm), ne, ctypes.byref(ty)))
            out.append((nm.value.decode(), tuple(ne), ty.value))
        return out

    def read(self, name, as_f32=True):
        """the tensor as f32 (numpy, shape = reversed ggml ne) or its stored bytes (uint8)"""
        import numpy as np
        ne, ty = (ctypes.c_int64 * 4)(), ctypes.c_int()
        rc = load().tsk_gguf_find_tensor(self.h, name.encode(), ne, ctypes.byref(ty))
        if rc < 0:
            check(rc)
        n = ne[0] * ne[1] * ne[2] * ne[3]
        if as_f32:
            out = np.empty(n, np.float32)
        else:
            nb = {0: 4 * n, 1: 2 * n, 30: 2 * n, 8: 34 * (n // 32)}.get(ty.value, 0)
            out = np.empty(nb, np.uint8)
        check(load().tsk_gguf_read_tensor(self.h, name.encode(), int(as_f32), out.ctypes.data, out.nbytes))
        if not as_f32:
            return out
        dims = list(ne)
        while len(dims) > 1 and dims[-1] == 1:
            dims.pop()
        return out.reshape(tuple(reversed(dims)))

    def u32(self, key):
        v = ctypes.c_uint32()
        check(load().tsk_gguf_get_u32(self.h, key.encode(), ctypes.byref(v)))
        return v.value

    def f32(self, key):
        v = ctypes.c_float()
        check(load().tsk_gguf_get_f32(self.h, key.encode(), ctypes.byref(v)))
        return v.value

    def str(self, key):
        v = ctypes.c_char_p()
        check(load().tsk_gguf_get_str(self.h, key.encode(), ctypes.byref(v)))
        return v.value.decode()

    def dit_config(self, **kw):
        c = dit_config(**kw)
        check(load().tsk_dit_config_from_gguf(self.h, ctypes.byref(c)))
        return c

    def t5_config(self, **kw):
        c = t5_config(**kw)
        check(load().tsk_t5_config_from_gguf(self.h, ctypes.byref(c)))
        return c

    def mmdit_config(self, **kw):
        """the reference graph's sizes from the file; kw (capacities) applied after"""
        c = mmdit_config()
        check(load().tsk_mmdit_config_from_gguf(self.h, ctypes.byref(c)))
        for k_, v_ in kw.items():
            setattr(c, k_, v_)
        return c

    def load_into(self, model):
        """all weights of a Dit or T5 driver from this file"""
        fn = load().tsk_dit_load_gguf if isinstance(model, Dit) else load().tsk_t5_load_gguf
        check(fn(model.h, self.h))
