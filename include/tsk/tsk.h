/*
 * tsk.h — C ABI of the MI355X (gfx950) MM-DiT hot path.
 *
 * The entry points mirror the ggml operator nodes that thinksound.cpp's MM-DiT
 * graph builder emits, so a ggml backend (or any C caller) can hand those nodes
 * to these kernels 1:1:
 *
 *   tsk_mul_mat         <- ggml_mul_mat(ctx, W, x)            src/mmdit.cpp:13, :24
 *                          (+ the ggml_add bias node of lin()  src/mmdit.cpp:14)
 *   tsk_flash_attn_ext  <- ggml_flash_attn_ext(ctx,q,k,v,mask,scale,max_bias,softcap)
 *                          + ggml_flash_attn_ext_set_prec     src/mmdit.cpp:91-92
 *   tsk_rms_norm_mul    <- ggml_mul(ggml_rms_norm(x, eps), w)  src/mmdit.cpp:78-80
 *   tsk_rope_ext        <- ggml_rope_ext(..., GGML_ROPE_TYPE_NORMAL, ...) src/mmdit.cpp:96-99
 *   tsk_qk_norm_rope    <- the chain rms_norm -> mul(w) -> rope_ext of
 *                          pre_attn                             src/mmdit.cpp:221-223
 *   tsk_norm            <- ggml_norm(x, eps)                   src/mmdit.cpp:59
 *   tsk_im2col_1d       <- ggml_im2col(w, x, s0,0,p0,0,d0,0, false, type) src/mmdit.cpp:21
 *   tsk_conv1d          <- conv_cl / conv1d_f32                src/mmdit.cpp:20-34
 *   tsk_swiglu          <- ggml_mul(ggml_silu(h1), h3)         src/mmdit.cpp:42, :50
 *   tsk_conv_mlp_swiglu <- convmlp                             src/mmdit.cpp:39-44
 *   tsk_mlp_swiglu      <- mlp                                 src/mmdit.cpp:47-52
 *   tsk_dit_*           <- ts_dit::load / forward / sample     src/mmdit.h:9-42
 *                          (the benchmarked two-stream block shape)
 *   tsk_mmdit_*         <- ts_dit::forward / sample, the reference's own
 *                          three-stream graph                   src/mmdit.cpp:119-376
 *   tsk_t5_attention    <- mul_mat(k,q) + bias + pad -> soft_max -> mul_mat
 *                                                              src/t5_encoder.cpp:68-73
 *   tsk_t5_*            <- ts_t5::load / encode                src/t5_encoder.cpp:28-104
 *   tsk_vae_*           <- ts_vae::load / decode               src/vae_decoder.cpp:7-124
 *
 * Conventions (all follow ggml):
 *   - tensors are non-owning views: ne[] = extents with ne[0] fastest,
 *     nb[] = byte strides, data = DEVICE pointer (tsk_dit_* host entry points
 *     say so explicitly where they take host memory);
 *   - type ids use ggml's enum ggml_type numbering;
 *   - every entry point validates shapes, types, strides and pointers on the
 *     host BEFORE any launch and returns a negative tsk_status instead of
 *     aborting (ggml would GGML_ASSERT);
 *   - kernels are enqueued on the given stream (a hipStream_t; NULL = the
 *     null stream) and are not synchronised; entry points are reentrant per
 *     stream: calls on different streams may run concurrently from different
 *     host threads (one stream per caller thread, as a ggml backend uses it);
 *   - operators that need device scratch take it from the workspace of their
 *     stream: a buffer the caller binds with tsk_set_workspace (sized with
 *     tsk_workspace_size; the library then never allocates), or else one the
 *     library owns per (device, stream) and grows on first need (that growth
 *     waits for the stream and reallocates; once every shape has been seen
 *     no operator allocates or synchronises).
 */
#ifndef TSK_TSK_H
#define TSK_TSK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (values of ggml's enum ggml_type). */
enum tsk_type {
    TSK_TYPE_F32  = 0,
    TSK_TYPE_F16  = 1,
    TSK_TYPE_Q8_0 = 8,   /* blocks of {fp16 d; int8 qs[32]} (34 bytes) along ne[0] */
    TSK_TYPE_I32  = 26,
    TSK_TYPE_BF16 = 30,
    /* Extension (no ggml counterpart): Q8_0 weights repacked once for the GPU
     * by tsk_q8_0_repack. Same values as TSK_TYPE_Q8_0, split into two planes:
     * int8 qs[ne1][ne0] followed by fp16 d[ne1][ne0/32]; nb[] are ignored. */
    TSK_TYPE_Q8_0_SPLIT = 0x1008
};

/* ggml_prec values (ggml_flash_attn_ext_set_prec). */
enum tsk_prec {
    TSK_PREC_DEFAULT = 0,
    TSK_PREC_F32     = 10
};

/* ggml_rope_type: only NORMAL (adjacent pairs) is on the MM-DiT path. */
enum tsk_rope_mode {
    TSK_ROPE_TYPE_NORMAL = 0
};

enum tsk_status {
    TSK_OK               = 0,
    TSK_ERR_INVALID_ARG  = -1,  /* null pointer, bad scalar argument      */
    TSK_ERR_TYPE         = -2,  /* element type not supported             */
    TSK_ERR_SHAPE        = -3,  /* ne[] inconsistent between operands     */
    TSK_ERR_STRIDE       = -4,  /* nb[] layout not supported              */
    TSK_ERR_ALIGN        = -5,  /* pointer / row alignment not supported  */
    TSK_ERR_UNSUPPORTED  = -6,  /* valid ggml node this library does not run */
    TSK_ERR_NOT_INIT     = -7,  /* tsk_init was not called                */
    TSK_ERR_HIP          = -8,  /* a HIP runtime call failed              */
    TSK_ERR_NOMEM        = -9   /* device allocation failed               */
};

typedef struct tsk_tensor {
    int32_t type;      /* enum tsk_type                          */
    int64_t ne[4];     /* extents, ne[0] fastest                 */
    size_t  nb[4];     /* byte strides (nb[0] = element/block size) */
    void   *data;      /* device pointer                         */
} tsk_tensor;

typedef void *tsk_stream;   /* hipStream_t */

/* ---- library ---------------------------------------------------------- */

/* Select the HIP device, read its limits (CU count, LDS per workgroup) and
 * the launch-shape overrides of tuning sweeps (TSK_* environment variables,
 * read here and never on a launch). Idempotent; a later call re-reads them,
 * so it must not run while other threads have operators in flight.
 * Operators are reentrant across streams; a model object (tsk_dit, tsk_mmdit,
 * tsk_t5, tsk_vae) owns its activations and runs one call at a time in its
 * stream's order -- concurrent callers use one model per stream. */
int         tsk_init(int device);
/* Release library-owned device memory (workspaces). */
int         tsk_shutdown(void);
/*
 * Bind a caller-owned device buffer (256-byte aligned) as the workspace of
 * every operator enqueued on `stream` on the current device; ptr = NULL,
 * bytes = 0 unbinds. An operator whose scratch exceeds `bytes` returns
 * TSK_ERR_NOMEM. The buffer must stay valid while work queued on the stream
 * may read it. No counterpart in ggml (whose backends keep scratch pools):
 * for callers that cannot let a library allocate.
 */
int         tsk_set_workspace(tsk_stream stream, void *ptr, size_t bytes);
/* Free the library-owned workspace of `stream` (call before destroying a
 * stream that operators ran on; waits for it). */
int         tsk_release_workspace(tsk_stream stream);
/* Text for a tsk_status value. */
const char *tsk_status_string(int status);
/* Detail of the last error reported on the calling thread ("" if none). */
const char *tsk_last_error(void);
/* Library version string. */
const char *tsk_version(void);

/* ---- operators -------------------------------------------------------- */

/*
 * dst = a x b (+ bias), ggml_mul_mat semantics.
 *   a    : weight, ne = [K, M, 1, 1]; F32, F16, BF16, Q8_0 or Q8_0_SPLIT.
 *          Rows must be contiguous (nb[0] = element/block size).
 *   b    : activations, ne = [K, N, n2, n3]; F32 (or BF16), rows contiguous.
 *          As in ggml, b is first converted to a's vec_dot type: BF16 weights
 *          round b to bf16 (RNE); Q8_0 weights quantize b per 32-block to Q8_0
 *          (amax/127 scale, round-to-nearest-even); F16 weights round to fp16.
 *   bias : nullable, F32 ne = [M]; fused ggml_add broadcast over N.
 *   dst  : F32 (or BF16), ne = [M, N, n2, n3]; rows contiguous.
 * K must be a multiple of 32 for Q8_0 (ggml block) and of 8 otherwise.
 */
int tsk_mul_mat(const tsk_tensor *a, const tsk_tensor *b, const tsk_tensor *bias,
                tsk_tensor *dst, tsk_stream stream);

/*
 * tsk_mul_mat that allocates nothing: no counterpart in the reference (ggml's
 * backends own their scratch pools). For callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. Same operands, semantics and results (bit for bit) as
 * tsk_mul_mat; its scratch (the bf16 rows of f32 activations, the Q8_0
 * repack and activation planes) lives in one fixed array of
 * TSK_MUL_MAT_NOALLOC_SCRATCH bytes per GPU, resident until the process
 * ends; a node needing more (tsk_workspace_size) returns TSK_ERR_NOMEM
 * before any launch. Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (other streams or threads) race.
 */
#define TSK_MUL_MAT_NOALLOC_SCRATCH (32u << 20)
int tsk_mul_mat_noalloc(const tsk_tensor *a, const tsk_tensor *b, const tsk_tensor *bias,
                        tsk_tensor *dst, tsk_stream stream);

/*
 * ggml_flash_attn_ext semantics (non-causal, online softmax):
 *   q    : ne = [D, Nq, H, B]   F32, F16 or BF16
 *   k    : ne = [D, Nkv, Hkv, B] F32, F16 or BF16   (H % Hkv == 0)
 *   v    : ne = [D, Nkv, Hkv, B] same type as k
 *   mask : nullable, F16 (or F32) ne = [Nkv, >=Nq, m2, m3]; added as
 *          slope*mask; broadcast over heads/batch when m2 | H, m3 | B.
 *   dst  : F32 (or BF16) ne = [D, H, Nq, B]  (ggml's permuted result)
 * D must be 64. Q is converted to K's type as ggml-cpu does (F16/BF16 K);
 * products are exact, logits/softmax/accumulation are fp32; V of a 16-bit
 * type is used as fp16 in the P.V product (the same cast mmdit.cpp:89-90
 * applies before the node). With F32 K/V everything is fp32.
 * prec: TSK_PREC_DEFAULT or TSK_PREC_F32 (both run fp32 softmax).
 * Scratch: BF16 V of the unmasked 16-bit path is transposed to fp16 in the
 * stream's workspace first; F16 V (the node mmdit.cpp:88-92 emits) and the
 * other paths take none.
 */
int tsk_flash_attn_ext(const tsk_tensor *q, const tsk_tensor *k, const tsk_tensor *v,
                       const tsk_tensor *mask, float scale, float max_bias,
                       float logit_softcap, int prec, tsk_tensor *dst,
                       tsk_stream stream);

/*
 * The T5 encoder's self-attention chain (src/t5_encoder.cpp:68-73): scores =
 * mul_mat(k, q) (no 1/sqrt(d): scale 1 there) + the relative-position bias
 * rel_bias[bucket(k - q)][h] (:69, :95) + the padding mask (-inf on keys
 * whose token id is 0, :70, :97) -> soft_max -> mul_mat(v^T, .), run as one
 * flash attention whose bias comes from a per-head table over k - q:
 *   q, k, v  : F32 ne = [64, n, H, 1], rows 16-byte aligned
 *   rel_lut  : F32 ne = [2 n_max - 1, H], n_max >= n, rows contiguous:
 *              rel_lut[h][n_max - 1 + k - q] is the bias of key k for query q
 *   key_valid: DEVICE uint8 [n], 0 marks a padded key (its weight is 0)
 *   dst      : F32 ne = [64, H, n, 1] (ggml's permuted result)
 * A row whose keys are all padded gives 0 (ggml: 0/0 guarded as 0).
 */
int tsk_t5_attention(const tsk_tensor *q, const tsk_tensor *k, const tsk_tensor *v,
                     const tsk_tensor *rel_lut, const uint8_t *key_valid, float scale,
                     tsk_tensor *dst, tsk_stream stream);

/* dst = rms_norm(x, eps) * w   over ne[0] of x (F32/BF16 in, same type out);
 * w F32 ne = [ne0]. */
int tsk_rms_norm_mul(const tsk_tensor *x, const tsk_tensor *w, float eps,
                     tsk_tensor *dst, tsk_stream stream);

/*
 * T5's pre-projection norm and the conversion of the Q8_0 mul_mat that
 * follows it (src/t5_encoder.cpp:58-61, :79-81): dst = Q8_0 quantization
 * (tsk_q8_0_quantize's rounding) of rms_norm(x, eps) * w, in one pass over
 * the row -- the same bits as tsk_rms_norm_mul followed by tsk_q8_0_quantize.
 * x F32 ne = [n, rows] (n = 1024, 2048 or 4096; rows 16-byte aligned), w F32
 * [n], dst Q8_0 of x's shape (nb[0] = 34). Scratch: the stream's workspace.
 */
int tsk_rms_norm_q8_0(const tsk_tensor *x, const tsk_tensor *w, float eps, tsk_tensor *dst,
                      tsk_stream stream);

/* dst = layer norm (no affine) of x over ne[0], eps as ggml_norm. F32/BF16. */
int tsk_norm(const tsk_tensor *x, float eps, tsk_tensor *dst, tsk_stream stream);

/*
 * ggml_rope_ext, mode NORMAL, on x ne = [n_dims_total, n_head, S, B] F32/BF16
 * with pos I32 ne = [S]. theta_i = pos * freq_base^(-2i/n_dims) built by the
 * same running product as ggml-cpu's rope cache, times freq_scale.
 * ext_factor must be 0 and attn_factor 1 (the MM-DiT call, mmdit.cpp:98).
 */
int tsk_rope_ext(const tsk_tensor *x, const tsk_tensor *pos, int n_dims, int mode,
                 float freq_base, float freq_scale, float ext_factor,
                 float attn_factor, tsk_tensor *dst, tsk_stream stream);

/*
 * Fused pre_attn prologue: dst = rope_ext(rms_norm(x, eps) * w, pos) with
 * pos == NULL meaning "no RoPE" (text stream, mmdit.cpp:223).
 * x ne = [64, n_head, S, B] F32/BF16, w F32 [64]; dst F32/BF16 same shape.
 */
int tsk_qk_norm_rope(const tsk_tensor *x, const tsk_tensor *w, const tsk_tensor *pos,
                     float eps, int n_dims, float freq_base, float freq_scale,
                     tsk_tensor *dst, tsk_stream stream);

/* Quantize F32 rows (ne0 % 32 == 0) to Q8_0 with ggml-cpu's x86 rounding
 * (d = amax/127 stored fp16, q = rne(x*127/amax)). dst type Q8_0. */
int tsk_q8_0_quantize(const tsk_tensor *x, tsk_tensor *dst, tsk_stream stream);
/* Dequantize Q8_0 or Q8_0_SPLIT to F32: y = fp32(d) * q (exact). */
int tsk_q8_0_dequantize(const tsk_tensor *x, tsk_tensor *dst, tsk_stream stream);
/* Repack ggml Q8_0 blocks into the TSK_TYPE_Q8_0_SPLIT planes (bit-preserving).
 * dst->data must hold ne1*ne0 + 2*ne1*(ne0/32) bytes. */
int tsk_q8_0_repack(const tsk_tensor *src, tsk_tensor *dst, tsk_stream stream);
/* Bytes a Q8_0_SPLIT tensor of ne = [K, M] occupies. */
size_t tsk_q8_0_split_nbytes(int64_t K, int64_t M);

/* ---- convolution and SwiGLU glue (src/mmdit.cpp:20-52) -------------------
 * The reference graph's latent / clip streams run kernel-3 convolutions
 * (conv1d_f32 = ggml_im2col + ggml_mul_mat, conv_cl, convmlp) and its text
 * stream SwiGLU linear MLPs (mlp). Convolutions here are one GEMM with
 * K = KW * IC over an implicit im2col (the GEMM gathers shifted input rows
 * while staging them; no im2col buffer), which needs the kernel's K in
 * kw-major order: tsk_conv1d_pack_weight writes that layout once at load,
 * and other layouts are permuted into library scratch on every call. Type
 * rules are ggml_mul_mat's: BF16 kernels round the input to bf16 (RNE) and
 * sum exact products in fp32; F32 kernels (the Q8_0 DiT keeps its 3-D
 * kernels in F32) run all-fp32. Only the fp32 summation order differs from
 * the ggml graph. */

/*
 * ggml_im2col(kernel, x, s0, 0, p0, 0, d0, 0, false, dst type), 1-D
 * (conv1d_f32, src/mmdit.cpp:21):
 *   kernel : ne = [KW, IC, ...]; only its shape is read
 *   x      : F32 ne = [IW, IC, N, 1], any element strides (a ggml_transpose
 *            view of a channels-fastest [IC, IW] tensor included)
 *   dst    : ne = [IC * KW, OW, N, 1] F32, F16 or BF16, rows contiguous,
 *            OW = (IW + 2 p0 - d0 (KW - 1) - 1) / s0 + 1
 *   dst[n][ow][ic * KW + kw] = x[n][ic][ow * s0 + kw * d0 - p0], 0 outside [0, IW).
 */
int tsk_im2col_1d(const tsk_tensor *kernel, const tsk_tensor *x, int s0, int p0, int d0,
                  tsk_tensor *dst, tsk_stream stream);

/*
 * conv_cl (src/mmdit.cpp:28-34): channels-last 1-D convolution,
 *   dst[b][ow][oc] = bias[oc] + sum_{ic,kw} w[oc][ic][kw] x[b][ow s0 + kw d0 - p0][ic]
 *   w    : ne = [KW, IC, OC] BF16 or F32, any element strides; the kw-major
 *          storage nb = [IC es, es, >= KW IC es (16-B multiple)] is read in
 *          place (tsk_conv1d_pack_weight), other layouts are permuted into
 *          scratch per call
 *   bias : nullable F32 [OC], contiguous, 16-B aligned
 *   x    : ne = [IC, IW, B, 1] F32, or BF16 with BF16 w (the canonical
 *          channels-fastest layout: the reference's transpose is implicit);
 *          rows contiguous, nb[1], nb[2] and data 16-B aligned; IC % 8 == 0
 *   dst  : ne = [OC, OW, B, 1] F32 or BF16, rows contiguous and uniformly
 *          strided (nb[2] = OW nb[1])
 */
int tsk_conv1d(const tsk_tensor *w, const tsk_tensor *bias, const tsk_tensor *x, int s0,
               int p0, int d0, tsk_tensor *dst, tsk_stream stream);

/* Copy a conv kernel ne = [KW, IC, OC] (any strides, BF16 or F32) into dst of
 * the same type and shape laid out kw-major: nb = [IC es, es, KW IC es, ...]
 * (a load-time permutation, like tsk_q8_0_repack; bit-preserving). */
int tsk_conv1d_pack_weight(const tsk_tensor *w, tsk_tensor *dst, tsk_stream stream);

/* dst = ggml_mul(ggml_silu(a), b) (src/mmdit.cpp:42, :50), F32, all three
 * contiguous and of one shape; silu(a) = a / (1 + exp(-a)). */
int tsk_swiglu(const tsk_tensor *a, const tsk_tensor *b, tsk_tensor *dst, tsk_stream stream);

/*
 * convmlp (src/mmdit.cpp:39-44): dst = conv(w2, silu(conv(w1, x)) * conv(w3, x)),
 * every conv stride 1, padding 1, dilation 1, no bias. w1, w3: [KW, IC, HID],
 * w2: [KW, HID, OC], all BF16 or all F32 (layouts as tsk_conv1d); x and dst
 * as tsk_conv1d; HID % 8 == 0. BF16: w1 and w3 run as ONE GEMM whose epilogue
 * writes silu(h1) * h3 rounded to bf16 -- the conversion ggml_mul_mat applies
 * to it before w2 -- so the hidden state is written once; F32: two GEMMs and
 * tsk_swiglu. The hidden state lives in library scratch.
 */
int tsk_conv_mlp_swiglu(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2,
                        const tsk_tensor *x, tsk_tensor *dst, tsk_stream stream);

/* mlp (src/mmdit.cpp:47-52): dst = w2 (silu(w1 x) * w3 x), linear layers
 * without bias: w1, w3 ne = [IC, HID], w2 ne = [HID, OC], all BF16 or all
 * F32, rows contiguous; x ne = [IC, N, n2, n3] F32 (or BF16 with BF16 weights),
 * dst [OC, N, n2, n3] F32 or BF16, rows of both uniformly strided. */
int tsk_mlp_swiglu(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2,
                   const tsk_tensor *x, tsk_tensor *dst, tsk_stream stream);

/* ggml_op ids used by tsk_supports_op (values of ggml's enum ggml_op are not
 * stable across ggml revisions, so these are this library's own). */
enum tsk_op {
    TSK_OP_MUL_MAT        = 1,
    TSK_OP_FLASH_ATTN_EXT = 2,
    TSK_OP_RMS_NORM_MUL   = 3,
    TSK_OP_ROPE_EXT       = 4,
    TSK_OP_NORM           = 5,
    TSK_OP_IM2COL         = 6,   /* srcs: kernel, x; fixed s0 = 1, p0 = 1, d0 = 1 */
    TSK_OP_CONV1D         = 7,   /* srcs: w, x, bias; fixed s0 = 1, p0 = 1, d0 = 1 */
    TSK_OP_CONV_MLP_SWIGLU = 8,  /* srcs: w1, w3, w2, x */
    TSK_OP_MLP_SWIGLU     = 9,   /* srcs: w1, w3, w2, x */
    TSK_OP_RMS_NORM_Q8_0  = 10   /* srcs: x, w */
};
/* Mirror of a ggml backend's supports_op: 1 if tsk would run the node with
 * these operand descriptors (data pointers are not inspected), else 0.
 * srcs follow the argument order of the matching entry point. */
int tsk_supports_op(int op, const tsk_tensor *const *srcs, int n_srcs,
                    const tsk_tensor *dst);
/* Device scratch (bytes) the node needs from its stream's workspace
 * (tsk_set_workspace); 0 for operators that need none. Validates the
 * descriptors like the entry point (data pointers are not inspected) and
 * returns its status. Counterpart of a ggml backend's buffer sizing
 * (ggml_backend_buft_get_alloc_size); srcs as for tsk_supports_op. */
int tsk_workspace_size(int op, const tsk_tensor *const *srcs, int n_srcs,
                       const tsk_tensor *dst, size_t *bytes);

/* ---- GGUF ingestion (ts_model::load_backend, src/common/ts_model.cpp:13-41) --
 * A host-side reader of the GGUF v2/v3 files the converters write
 * (convert/convert_thinksound.py, convert/convert_t5.py, convert/quantize_gguf.py)
 * and loaders that hand their tensors to the drivers by name. Tensor types
 * read: F32, F16, BF16, Q8_0 (others give TSK_ERR_TYPE). No GPU work except
 * inside the *_load_gguf calls (through the drivers' set_tensor). */
typedef struct tsk_gguf tsk_gguf;
int  tsk_gguf_open(const char *path, tsk_gguf **out);
void tsk_gguf_close(tsk_gguf *g);
int  tsk_gguf_n_tensors(const tsk_gguf *g);
int  tsk_gguf_tensor_info(const tsk_gguf *g, int i, const char **name, int64_t ne[4], int *type);
/* index of the tensor (>= 0) and its ggml ne / type, or a negative status */
int  tsk_gguf_find_tensor(const tsk_gguf *g, const char *name, int64_t ne[4], int *type);
/* the tensor's bytes as stored (as_f32 = 0) or converted to f32 (as_f32 = 1:
 * F16 / BF16 exactly, Q8_0 as fp32(d) * q); dst_bytes must match exactly */
int  tsk_gguf_read_tensor(const tsk_gguf *g, const char *name, int as_f32, void *dst, size_t dst_bytes);
/* metadata: integers / bools as u32, numbers as f32, strings (pointer valid
 * until tsk_gguf_close) */
int  tsk_gguf_get_u32(const tsk_gguf *g, const char *key, uint32_t *out);
int  tsk_gguf_get_f32(const tsk_gguf *g, const char *key, float *out);
int  tsk_gguf_get_str(const tsk_gguf *g, const char *key, const char **out);

/* ---- T5 encoder stack (counterpart of ts_t5, src/t5_encoder.cpp:28-104) -- */

typedef struct tsk_t5 tsk_t5;

typedef struct tsk_t5_config {
    int   d_model;       /* 2048 (GGUF t5.d_model, t5_encoder.cpp:32)      */
    int   d_ff;          /* 5120 (t5.d_ff)                                 */
    int   n_layers;      /* 24   (t5.n_layers, :33)                        */
    int   n_heads;       /* 32   (t5.n_heads)                              */
    int   d_kv;          /* 64   (t5.d_kv, :34; must be 64)                */
    int   rel_buckets;   /* 32   (t5.rel_buckets, :35)                     */
    int   rel_max_dist;  /* 128  (t5.rel_max_dist)                         */
    int   weight_type;   /* TSK_TYPE_Q8_0: every matrix a ggml Q8_0 tensor */
    int   max_tokens;    /* capacity: tokens per encode                    */
    float eps;           /* 1e-6 (t5.eps, :36)                             */
} tsk_t5_config;

/* Fill the T5-v1.1-xl defaults above (max_tokens 512). */
void tsk_t5_default_config(tsk_t5_config *cfg);
int  tsk_t5_create(const tsk_t5_config *cfg, tsk_t5 **out);
void tsk_t5_destroy(tsk_t5 *t5);
/* Named weights (the converter's names: rel_bias, blk.<i>.attn_norm, .q, .k,
 * .v, .o, .ffn_norm, .wi_0, .wi_1, .wo, out_norm) with their ggml shape and
 * type (TSK_TYPE_Q8_0 matrices, TSK_TYPE_F32 vectors and rel_bias). */
int  tsk_t5_n_tensors(const tsk_t5 *t5);
int  tsk_t5_tensor_info(const tsk_t5 *t5, int i, const char **name, int64_t ne[4], int *type);
/* Upload one weight from HOST memory in its stored form: ggml Q8_0 blocks
 * (34 bytes per 32 values along ne[0]) or F32; nbytes must match exactly. */
int  tsk_t5_set_tensor(tsk_t5 *t5, const char *name, const void *host_data, size_t nbytes);
/*
 * The encoder layers of ts_t5::encode (t5_encoder.cpp:56-88) on n <= max_tokens
 * embedded tokens (the tok_emb row gather, :46, stays with the caller), all
 * pointers HOST: x [n, d_model] f32, ids [n] (id 0 marks a padded key, :97)
 * -> out [n, d_model] f32 (after out_norm). Attention runs as
 * flash_attn_ext with the per-head relative-position bias + padding as its
 * additive F32 mask, scale 1 (the reference's mul_mat/add/soft_max/mul_mat
 * chain, :68-73).
 */
int  tsk_t5_encode(tsk_t5 *t5, int n, const float *x, const int32_t *ids, float *out,
                   tsk_stream stream);
/* Same with DEVICE x / out (f32) and HOST ids; no host synchronisation. */
int  tsk_t5_encode_device(tsk_t5 *t5, int n, const float *x_d, const int32_t *ids_host,
                          float *out_d, tsk_stream stream);
/* Layers [layer_begin, layer_end) only, then out_norm if final_norm (else the
 * residual stream itself): a stack split into stages, e.g. to check or
 * pipeline it layer by layer. HOST (encode_range) or DEVICE (encode_layers)
 * x / out; ids always HOST. */
int  tsk_t5_encode_range(tsk_t5 *t5, int n, const float *x, const int32_t *ids, int layer_begin,
                         int layer_end, int final_norm, float *out, tsk_stream stream);
int  tsk_t5_encode_layers(tsk_t5 *t5, int n, const float *x_d, const int32_t *ids_host,
                          int layer_begin, int layer_end, int final_norm, float *out_d,
                          tsk_stream stream);
/* t5.* metadata (t5_encoder.cpp:31-36) over the values already in cfg */
int  tsk_t5_config_from_gguf(const tsk_gguf *g, tsk_t5_config *cfg);
/* every weight by name from a GGUF file, in its stored type (Q8_0 / F32) */
int  tsk_t5_load_gguf(tsk_t5 *t5, const tsk_gguf *g);

/* ---- MM-DiT step driver (counterpart of ts_dit, src/mmdit.h:9-42) ------ */

typedef struct tsk_dit tsk_dit;

enum tsk_mlp_kind {
    TSK_MLP_GELU_TANH = 0   /* Linear(d, r*d) -> GELU(tanh) -> Linear(r*d, d) */
};

typedef struct tsk_dit_config {
    int   hidden;        /* 1024 */
    int   n_head;        /* 16   */
    int   head_dim;      /* 64   */
    int   depth;         /* 21 = joint + fused */
    int   fused_depth;   /* 14   */
    int   latent_dim;    /* 64   */
    int   text_seq;      /* 77   */
    int   mlp_hidden;    /* 4096 */
    int   mlp_kind;      /* enum tsk_mlp_kind */
    int   weight_type;   /* TSK_TYPE_BF16, or TSK_TYPE_Q8_0: the block
                            projections (attn.qkv, linear1, ffn.fc1, ffn.fc2)
                            as Q8_0 with Q8_0-quantized activations (ggml's
                            Q8_0 x Q8_0 mul_mat); every other matrix BF16 */
    int   max_batch;     /* capacity: batch rows per forward (2 for CFG) */
    int   max_latent;    /* capacity: latent tokens T                    */
    float rope_theta;    /* 10000 */
    float t_max_period;  /* 1     */
    float ln_eps;        /* 1e-5  (mmdit.cpp:59)  */
    float qk_eps;        /* 1e-6  (mmdit.cpp:10)  */
} tsk_dit_config;

/* Fill the 9 s / 30 s MM-DiT defaults above. */
void tsk_dit_default_config(tsk_dit_config *cfg);
/* Allocate device state for cfg (weights are zero until set). */
int  tsk_dit_create(const tsk_dit_config *cfg, tsk_dit **out);
void tsk_dit_destroy(tsk_dit *dit);
/* Number of named weight tensors and the i-th name / ggml shape. */
int  tsk_dit_n_tensors(const tsk_dit *dit);
int  tsk_dit_tensor_info(const tsk_dit *dit, int i, const char **name, int64_t ne[4]);
/* Upload one named weight from HOST f32 data, converted to the type the
 * driver stores it in: BF16 (RNE) matrices, F32 vectors, and for the Q8_0
 * driver's block projections ggml's reference Q8_0 quantization
 * (quantize_row_q8_0_ref; the converter's gguf-py quantize is bit-identical,
 * convert/quantize_gguf.py:41). */
int  tsk_dit_set_tensor(tsk_dit *dit, const char *name, const float *host_f32,
                        int64_t n_elements);
/* Upload a Q8_0 block projection of the Q8_0 driver from HOST ggml Q8_0
 * blocks as stored in a GGUF file (34 bytes per 32 values along ne[0],
 * nbytes exact): bit-preserving. TSK_ERR_TYPE for a tensor the driver does
 * not store as Q8_0. */
int  tsk_dit_set_tensor_q8_0(tsk_dit *dit, const char *name, const void *blocks, size_t nbytes);
/* The type the driver stores tensor i in: TSK_TYPE_BF16, TSK_TYPE_Q8_0 or
 * TSK_TYPE_F32 (a negative status for a bad index). */
int  tsk_dit_tensor_type(const tsk_dit *dit, int i);
/*
 * One flow evaluation for B (<= max_batch) rows, all pointers HOST, in the
 * layouts of ts_dit::forward (src/mmdit.h:26-29, src/mmdit.cpp:138, :289)
 * with the batch as the outermost dimension:
 *   latent ggml ne = [T, latent_dim, B]  (C order [B][latent_dim][T]),
 *   t [B], text ne = [hidden, text_seq, B]  (C order [B][text_seq][hidden])
 *   -> flow ne = [latent_dim, T, B]  (C order [B][T][latent_dim]).
 */
int  tsk_dit_forward(tsk_dit *dit, int B, int T, const float *latent, const float *t,
                     const float *text, float *flow, tsk_stream stream);
/* Same with DEVICE pointers for latent / text / flow (f32, same layouts) and
 * the B timesteps on the HOST (the t-embedding is built on the host in fp32
 * as mmdit.cpp:305-314 does); no host synchronisation. */
int  tsk_dit_forward_device(tsk_dit *dit, int B, int T, const float *latent_d,
                            const float *t_host, const float *text_d, float *flow_d,
                            tsk_stream stream);
/*
 * Rectified-flow Euler sampler with CFG (ts_dit::sample, mmdit.cpp:344-376),
 * cond/uncond batched as B=2 per step. HOST pointers, ts_dit::sample's
 * layouts (src/mmdit.h:31-33):
 *   noise ne = [T, latent_dim] (C order [latent_dim][T]),
 *   text_cond / text_uncond ne = [hidden, text_seq]
 *   -> out ne = [T, latent_dim]; flow0 (nullable, ne = [T, latent_dim]) =
 *   the CFG velocity of step 0.
 */
int  tsk_dit_sample(tsk_dit *dit, int T, const float *noise, const float *text_cond,
                    const float *text_uncond, int steps, float cfg_scale,
                    float *out, float *flow0, tsk_stream stream);
/* dit.* metadata of convert_thinksound.py:38-45 over the values already in cfg */
int  tsk_dit_config_from_gguf(const tsk_gguf *g, tsk_dit_config *cfg);
/* every weight by name from a GGUF file: Q8_0 tensors the driver stores as
 * Q8_0 bit for bit (tsk_dit_set_tensor_q8_0); F32 / F16 / BF16 tensors
 * converted to f32 and set as tsk_dit_set_tensor does; a Q8_0 tensor the
 * driver stores in another type returns TSK_ERR_TYPE (bf16(d * q) would not
 * be the Q8_0 x Q8_0 product the file asks for) */
int  tsk_dit_load_gguf(tsk_dit *dit, const tsk_gguf *g);

/*
 * Kernel timing of the step driver (extension, no counterpart in the
 * reference: ggml exposes no per-node timing). tsk_dit_timing(dit, 1) resets
 * the accumulators and records a HIP event pair around every launch of the
 * driver from then on (on the caller's stream); 0 stops recording.
 * tsk_dit_timing_read synchronises on the last event of `role` and returns the
 * summed kernel time, the number of launches and their algorithmic FLOPs and
 * bytes (weights + activations read + outputs written, once each).
 */
enum tsk_dit_role {
    TSK_ROLE_QKV = 0,        /* QKV projection GEMMs                      */
    TSK_ROLE_OUT = 1,        /* attention output projection (linear1)     */
    TSK_ROLE_FC1 = 2,        /* MLP up GEMM (+GELU)                       */
    TSK_ROLE_FC2 = 3,        /* MLP down GEMM (+gate*residual)            */
    TSK_ROLE_ATTN = 4,       /* flash attention                           */
    TSK_ROLE_ADALN = 5,      /* t_embed MLP + adaLN GEMVs                 */
    TSK_ROLE_OTHER = 6,      /* LN/modulate, QKV split, in/out projection */
    TSK_ROLE_COUNT = 7
};
int  tsk_dit_timing(tsk_dit *dit, int enable);
int  tsk_dit_timing_read(tsk_dit *dit, int role, double *ms, int64_t *launches,
                         double *flop, double *bytes);

/* ---- The reference's MM-DiT graph (ts_dit, src/mmdit.h:9-42) -------------
 * ts_dit::forward / ts_dit::sample as src/mmdit.cpp:119-376 builds them:
 * three streams (latent | clip | text) in 7 joint blocks, 14 fused blocks on
 * the latent, k3 convolutions (linear1, SwiGLU convMLP) on the latent and clip
 * streams, SwiGLU MLPs on text, per-token adaLN from extended_c (the sync
 * features interpolated to T plus global_c) on the latent stream and from
 * global_c on clip / text, a 154-token text stream (text_f padded to t5_dim
 * and concatenated with the T5 features), a k7 output convolution. Weights
 * by the converter's names (convert/convert_thinksound.py:32), each held in
 * one type and multiplied with ggml_mul_mat's semantics for it (src1
 * converted to the weight's vec_dot type): BF16 (input rounded to bf16),
 * F32, or Q8_0 (input quantized per 32 values, exact int32 block sums).
 * tsk_mmdit_create takes the types from cfg->weight_type, as the converters
 * write the files: TSK_TYPE_BF16 (convert/quantize_gguf.py --type bf16: BF16
 * linears and convolutions, the t_embed MLP F32), TSK_TYPE_Q8_0
 * (quantize_gguf.py, :9-15: 2-D linears with ne0 % 32 == 0 Q8_0, the 3-D
 * convolution kernels and "_emb" / "norm" / "empty" names F32) or
 * TSK_TYPE_F32 (the F32 GGUF); tsk_mmdit_create_from_gguf takes each
 * tensor's type from the file. sync_pos_emb, the learned empties and every
 * vector are F32. K / V are F16 in the attention (mmdit.cpp:89-90).
 * A model handles one call at a time, in its stream's order: it owns its
 * activations, staging and sampler state, so calls on one model from two
 * streams race; callers that need concurrency create a model per stream. */
typedef struct tsk_mmdit tsk_mmdit;

typedef struct tsk_mmdit_config {
    int   hidden;        /* 1024 (dit.hidden_dim)  */
    int   n_head;        /* 16   (head_dim 64)     */
    int   head_dim;      /* 64   */
    int   depth;         /* 21   */
    int   fused_depth;   /* 14   */
    int   latent_dim;    /* 64   */
    int   text_seq;      /* 77   (the text stream holds 2 text_seq tokens) */
    int   clip_dim;      /* 1024 */
    int   sync_dim;      /* 768  */
    int   t5_dim;        /* 2048 (text_f is zero-padded to this width, mmdit.cpp:179) */
    int   mlp_hidden;    /* 2816 (SwiGLU width of every MLP) */
    int   max_batch;     /* capacity: batch rows per forward (2 for CFG) */
    int   max_latent;    /* capacity: latent tokens T         */
    int   max_clip;      /* capacity: clip frames             */
    int   max_sync;      /* capacity: sync frames (multiple of 8) */
    float rope_theta;    /* 10000 */
    float t_max_period;  /* 1     */
    int   weight_type;   /* TSK_TYPE_BF16 (default), TSK_TYPE_Q8_0 or TSK_TYPE_F32: the
                            converters' storage rule tsk_mmdit_create applies */
} tsk_mmdit_config;

/* the reference's sizes (mmdit.h:17-22) and capacities for 30 s clips */
void tsk_mmdit_default_config(tsk_mmdit_config *cfg);
int  tsk_mmdit_create(const tsk_mmdit_config *cfg, tsk_mmdit **out);
void tsk_mmdit_destroy(tsk_mmdit *m);
int  tsk_mmdit_n_tensors(const tsk_mmdit *m);
/* name and ggml ne of tensor i: linear [in, out], conv [KW, IC, OC] */
int  tsk_mmdit_tensor_info(const tsk_mmdit *m, int i, const char **name, int64_t ne[4]);
/* the type the model holds tensor i in: TSK_TYPE_BF16, TSK_TYPE_F32 or TSK_TYPE_Q8_0 */
int  tsk_mmdit_tensor_type(const tsk_mmdit *m, int i);
/* Upload one weight from HOST f32 values in ggml / PyTorch memory order
 * (linear [out][in], conv [OC][IC][KW]); BF16 tensors are rounded RNE, Q8_0
 * tensors quantized with ggml's reference quantizer (quantize_row_q8_0_ref). */
int  tsk_mmdit_set_tensor(tsk_mmdit *m, const char *name, const float *host_f32, int64_t n);
/* Upload a Q8_0 tensor's blocks {fp16 d; int8 qs[32]} bit for bit (HOST,
 * rows in the file's order: ne[1] rows of ne[0] / 32 blocks). */
int  tsk_mmdit_set_tensor_q8_0(tsk_mmdit *m, const char *name, const void *blocks, size_t nbytes);
/* ts_dit::load (src/mmdit.cpp:104-116; ts_model::load_backend,
 * src/common/ts_model.cpp:13-41). tsk_mmdit_config_from_gguf reads the model
 * sizes from the dit.* keys of convert/convert_thinksound.py:38-45 (absent
 * keys keep *cfg's values), the SwiGLU width from audio_input_proj.2.w1, and
 * sets weight_type to the file's (Q8_0 if any tensor is Q8_0); capacities
 * stay the caller's. tsk_mmdit_create_from_gguf creates a model holding
 * every tensor in its file type (F32, BF16 or Q8_0; F16 matrices are
 * refused) and loads it. tsk_mmdit_load_gguf loads a file into a model whose
 * types it matches: Q8_0 blocks bit for bit, other types by value. */
int  tsk_mmdit_config_from_gguf(const tsk_gguf *g, tsk_mmdit_config *cfg);
int  tsk_mmdit_create_from_gguf(const tsk_gguf *g, const tsk_mmdit_config *cfg, tsk_mmdit **out);
int  tsk_mmdit_load_gguf(tsk_mmdit *m, const tsk_gguf *g);
/*
 * One flow evaluation for B (<= max_batch) rows, all pointers HOST, each
 * per-row block in the layout ts_dit::forward takes (src/mmdit.h:26-29,
 * src/mmdit.cpp:138-143), the batch outermost:
 *   latent ne = [T, latent_dim, B], t [B], clip_f ne = [clip_dim, clip_S, B],
 *   sync_f ne = [sync_dim, sync_S, B] (sync_S a multiple of 8),
 *   text_f ne = [clip_dim, text_seq, B], t5 ne = [t5_dim, text_seq, B],
 *   global_text ne = [clip_dim, B]  ->  flow ne = [latent_dim, T, B].
 */
int  tsk_mmdit_forward(tsk_mmdit *m, int B, int T, const float *latent, const float *t, int clip_S,
                       const float *clip_f, int sync_S, const float *sync_f, const float *text_f,
                       const float *t5, const float *global_text, float *flow, tsk_stream stream);
/* Same with DEVICE arrays (f32, the same layouts) for the inputs and flow,
 * t [B] on the HOST; no host synchronisation. */
int  tsk_mmdit_forward_device(tsk_mmdit *m, int B, int T, const float *latent_d, const float *t, int clip_S,
                              const float *clip_d, int sync_S, const float *sync_d, const float *text_d,
                              const float *t5_d, const float *global_text_d, float *flow_d, tsk_stream stream);
/*
 * Stage outputs (the dbg map of ts_dit::forward, src/mmdit.cpp:125, :333-336).
 * With tsk_mmdit_debug(m, 1) every forward keeps, in host memory, the
 * tensors the reference names x_in, t_emb, clip_pp, text_pp, clip_fc,
 * text_fc, gcmlp, global_c, extended_c, jb0_lat, jb0_clip, jb0_text (after
 * joint block 0; needs a fused block or a second joint block), after_joint,
 * after_fused: f32, ggml [H, S, B] (C order [B][S][H]). Each capture
 * synchronises the stream: a debugging aid, not for timed runs.
 * tsk_mmdit_debug_size returns the element count (negative status if the
 * last forward kept no such stage).
 */
int     tsk_mmdit_debug(tsk_mmdit *m, int enable);
int64_t tsk_mmdit_debug_size(const tsk_mmdit *m, const char *name);
int     tsk_mmdit_debug_get(const tsk_mmdit *m, const char *name, float *out, int64_t n);
/*
 * ts_dit::sample (src/mmdit.cpp:344-376): `steps` Euler steps of rectified
 * flow with CFG; each step runs the conditional and the unconditional
 * forward (empty_string_feat, empty_t5_feat, zero global text) as one B = 2
 * forward. HOST pointers in ts_dit::sample's layouts: noise / out ne =
 * [T, latent_dim]; flow0 (nullable) ne = [T, latent_dim], the CFG velocity of
 * step 0. Needs max_batch >= 2. The conditioning that does not depend on t
 * is computed once per call; the latent stays on the device between steps
 * and the CFG / Euler update runs there in the reference's rounding (the
 * same bits as a host loop over tsk_mmdit_forward).
 */
int  tsk_mmdit_sample(tsk_mmdit *m, int T, const float *noise, int clip_S, const float *clip_f, int sync_S,
                      const float *sync_f, const float *text_f, const float *t5, const float *global_text,
                      int steps, float cfg_scale, float *out, float *flow0, tsk_stream stream);

/* ---- Oobleck VAE decoder (ts_vae, src/vae_decoder.h:6-17) ---------------
 * ts_vae::decode (src/vae_decoder.cpp:62-124): conv k7 (latent_dim ->
 * 16 channels), 5 decoder blocks (SnakeBeta -> transposed conv of stride s,
 * kernel 2 s -> residual units of dilation 1, 3, 9: x + conv_k1(snake(
 * conv_k7_dil(snake(x))))), SnakeBeta -> conv k7 (no bias) -> out_channels.
 * SnakeBeta is y = x + sin^2(exp(alpha) x) exp(-beta) per channel
 * (:14-24). All weights and arithmetic F32 (the converter keeps the VAE F32,
 * convert/convert_vae.py:5): every convolution is an F32 x F32 ggml_mul_mat
 * (fp32 products and sums). The transposed convolutions take the converter's
 * conv1d kernels (flipped, channels swapped, convert/convert_vae.py:19-26) and
 * run as one 3-tap convolution whose output channels are the s phases of the
 * upsampled sequence -- the same sums as the reference's zero-stuffed conv1d
 * (:36-58) without its multiplications by the inserted zeros. */
typedef struct tsk_vae tsk_vae;

typedef struct tsk_vae_config {
    int latent_dim;      /* 64  (vae.latent_dim)   */
    int channels;        /* 128 (vae.channels)     */
    int out_channels;    /* 2   (vae.out_channels) */
    int c_mults[5];      /* 1, 2, 4, 8, 16 (vae.c_mults)  */
    int strides[5];      /* 2, 4, 4, 8, 8  (vae.strides)  */
    int max_latent;      /* capacity: latent frames per decode */
} tsk_vae_config;

/* the reference's configuration (convert/convert_vae.py:60-66), max_latent 646 */
void tsk_vae_default_config(tsk_vae_config *cfg);
int  tsk_vae_create(const tsk_vae_config *cfg, tsk_vae **out);
void tsk_vae_destroy(tsk_vae *v);
/* Named weights of the converter (decoder.layers.*; conv kernels ggml ne
 * [K, IC, OC], the transposed convolutions already as conv1d kernels;
 * vectors alpha / beta / bias), all F32. */
int  tsk_vae_n_tensors(const tsk_vae *v);
int  tsk_vae_tensor_info(const tsk_vae *v, int i, const char **name, int64_t ne[4]);
/* HOST f32 values in ggml / PyTorch memory order */
int  tsk_vae_set_tensor(tsk_vae *v, const char *name, const float *host_f32, int64_t n);
/* Upsampling factor: the product of the strides (2048). */
int  tsk_vae_hop(const tsk_vae *v);
/*
 * Decode T <= max_latent latent frames, HOST pointers in ts_vae's layouts
 * (src/vae_decoder.h:7-8): latent ne = [T, latent_dim] (C order
 * [latent_dim][T]) -> audio ne = [T_audio, out_channels] planar (C order
 * [out_channels][T_audio]), T_audio = T * hop. Returns TSK_OK or a negative
 * status; *t_audio receives T_audio.
 */
int  tsk_vae_decode(tsk_vae *v, int T, const float *latent, float *audio, int64_t *t_audio, tsk_stream stream);
/* Same with DEVICE latent / audio arrays; no host synchronisation. */
int  tsk_vae_decode_device(tsk_vae *v, int T, const float *latent_d, float *audio_d, tsk_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* TSK_TSK_H */
