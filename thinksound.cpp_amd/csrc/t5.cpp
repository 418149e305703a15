// t5.cpp — T5 encoder stack on gfx950 (counterpart of ts_t5::encode,
// src/t5_encoder.cpp:40-104): the configuration-4 workload (T5-v1.1-xl: 24
// layers, d_model 2048, 32 heads x 64, gated-GELU d_ff 5120, 32-bucket
// relative-position bias, Q8_0 weights).
//
// Per layer (t5_encoder.cpp:56-84), all activations f32 between ops:
//   h = rms_norm(x) * attn_norm                       rms_norm kernel
//   q | k | v = Q8_0 mul_mat(W_qkv, h)                h quantized to Q8_0 once,
//                                                     one int8-MFMA GEMM over the
//                                                     three weights stacked
//   o = flash_attn_ext(q, k, v, mask, scale 1)        mask[h][q][k] =
//                                                     rel_bias[bucket(k-q)][h] + pad[k],
//                                                     read from a per-head table
//                                                     over k - q and the key padding
//   x += Q8_0 mul_mat(W_o, o)                         residual in the epilogue
//   h = rms_norm(x) * ffn_norm
//   g = gelu(wi_0 h) * (wi_1 h)                       one GEMM over wi_0 / wi_1
//                                                     rows interleaved, GEGLU epilogue
//   x += Q8_0 mul_mat(wo, g)
// then out_norm. The reference adds the bias and the padding as two ggml_add
// nodes before its soft_max (:69-71); the padding is 0 or -inf, so one
// additive mask holds the same values. The attention adds, for key k of query
// q, lut[h][k - q + max_tokens - 1] + (valid[k] ? 0 : -inf): the same float a
// materialised [H][n][n] mask would hold, from a [H][2 max_tokens - 1] table
// instead of 33.5 MB per layer at 512 tokens. Bucket ids are computed on the
// host in double precision exactly as the reference does (:95); the device
// only gathers the bias table through them.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/tsk/tsk.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

using namespace tsk;

namespace {

struct T5W {
    std::string name;
    int64_t ne0, ne1;
    int type;              // TSK_TYPE_Q8_0 (matrices) or TSK_TYPE_F32
};

struct Layer {
    int8_t *qkv_q, *o_q, *wi_q, *wo_q;       // int8 planes [M][K]
    uint16_t *qkv_d, *o_d, *wi_d, *wo_d;     // fp16 scale planes [M][K / 32]
    float *attn_norm, *ffn_norm;
};

int hipcheck(hipError_t e, const char *what) { return e == hipSuccess ? TSK_OK : hip_fail(e, what); }

// t5_encoder.cpp:14-26 (host, double precision, as the reference)
int t5_bucket(int rel, int num_buckets, int max_dist) {
    int ret = 0;
    num_buckets /= 2;
    if (rel > 0) ret += num_buckets;
    const int n = std::abs(rel);
    const int max_exact = num_buckets / 2;
    if (n < max_exact) {
        ret += n;
    } else {
        const int v = max_exact + (int) (std::log((double) n / max_exact) / std::log((double) max_dist / max_exact) *
                                         (num_buckets - max_exact));
        ret += std::min(v, num_buckets - 1);
    }
    return ret;
}

}  // namespace

struct tsk_t5 {
    tsk_t5_config cfg;
    std::vector<T5W> w;
    std::unordered_map<std::string, int> idx;
    std::vector<Layer> layers;
    char *blob = nullptr;                    // every device weight
    float *rel_bias = nullptr, *out_norm = nullptr;
    // activations
    float *x = nullptr, *h = nullptr, *qkv = nullptr, *att = nullptr, *g = nullptr, *rel_lut = nullptr, *ones = nullptr;
    int8_t *qx = nullptr;
    float *dx = nullptr;
    int32_t *bkt = nullptr;                  // bucket of relative distance r at r + max_tokens - 1
    uint8_t *valid = nullptr;                // key valid flags
    float *io = nullptr;                     // host-entry staging (x in, out)
};

namespace {

// lut[h][r] = rel_bias[bkt[r]][h], r = k - q + maxn - 1 in [0, 2 maxn - 1)
__global__ void t5_lut_kernel(const float *rel_bias, const int32_t *bkt, int H, int maxn, float *lut) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int nr = 2 * maxn - 1;
    if (i >= (int64_t) H * nr) return;
    const int r = (int) (i % nr), h = (int) (i / nr);
    lut[i] = rel_bias[(int64_t) bkt[r] * H + h];
}

__global__ void fill_kernel(float *p, int64_t n, float v) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

int q8_gemm(tsk_t5 *t, const int8_t *qw, const uint16_t *dw, int N, int K, int M, int epi, float *y, int64_t ld_y,
            float *res, hipStream_t s) {
    GemmParams p;
    memset(&p, 0, sizeof(p));
    p.qw = qw; p.dw = dw; p.qx = t->qx; p.dx = t->dx;
    p.y = y; p.ld_y = ld_y; p.M = M; p.N = N; p.K = K; p.epi = epi;
    if (epi == EPI_GATE_RES) {
        p.res = res; p.ld_res = M;
        p.gate = t->ones; p.ld_gate = 0; p.rows_per_gate = N;    // gate = 1: a plain residual add
    }
    return hipcheck(launch_gemm_q8(p, s), "t5 q8 gemm");
}

int quantize(tsk_t5 *t, const float *x, int N, int K, hipStream_t s) {
    return hipcheck(launch_quantize_rows_q8(x, 1, K, N, K, t->qx, t->dx, s), "t5 quantize");
}

// rms_norm * w straight into the Q8_0 planes of the next GEMM's activations
// (the two-launch path when the fused kernel does not take the width)
int rmsnorm_q8(tsk_t5 *t, const float *x, const float *w, float eps, int N, int d, hipStream_t s);

int rmsnorm(const float *x, const float *w, float eps, int N, int d, float *y, hipStream_t s) {
    View4 a;
    memset(&a, 0, sizeof(a));
    a.data = (void *) x; a.type = TSK_TYPE_F32;
    a.ne[0] = d; a.ne[1] = N; a.ne[2] = a.ne[3] = 1;
    a.nb[0] = 4; a.nb[1] = (int64_t) d * 4; a.nb[2] = a.nb[3] = a.nb[1] * N;
    View4 o = a;
    o.data = y;
    return hipcheck(launch_rms_norm_mul(a, w, eps, o, s), "t5 rms_norm");
}

int rmsnorm_q8(tsk_t5 *t, const float *x, const float *w, float eps, int N, int d, hipStream_t s) {
    if (d == 1024 || d == 2048 || d == 4096)
        return hipcheck(launch_rms_norm_q8(x, d, w, eps, t->qx, t->dx, N, d, s), "t5 rms_norm + quantize");
    int rc = rmsnorm(x, w, eps, N, d, t->h, s);
    return rc ? rc : quantize(t, t->h, N, d, s);
}

}  // namespace

extern "C" void tsk_t5_default_config(tsk_t5_config *c) {
    if (!c) return;
    c->d_model = 2048; c->d_ff = 5120; c->n_layers = 24; c->n_heads = 32; c->d_kv = 64;
    c->rel_buckets = 32; c->rel_max_dist = 128; c->weight_type = TSK_TYPE_Q8_0; c->max_tokens = 512;
    c->eps = 1e-6f;
}

extern "C" void tsk_t5_destroy(tsk_t5 *t) {
    if (!t) return;
    (void) hipDeviceSynchronize();
    void *bufs[] = {t->blob, t->x, t->h, t->qkv, t->att, t->g, t->rel_lut, t->ones, t->qx, t->dx, t->bkt, t->valid, t->io};
    for (void *b : bufs)
        if (b) (void) hipFree(b);
    delete t;
}

extern "C" int tsk_t5_create(const tsk_t5_config *cfg, tsk_t5 **out) {
    if (!out || !cfg) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    *out = nullptr;
    const tsk_t5_config &c = *cfg;
    if (c.d_kv != 64) return fail(TSK_ERR_UNSUPPORTED, "d_kv must be 64");
    if (c.weight_type != TSK_TYPE_Q8_0) return fail(TSK_ERR_UNSUPPORTED, "T5 weights must be Q8_0");
    if (c.n_layers < 1 || c.n_heads < 1 || c.n_heads > 256 || c.max_tokens < 1 || c.max_tokens > 8192)
        return fail(TSK_ERR_SHAPE, "n_layers / n_heads / max_tokens");
    if (c.d_model % 32 || c.d_ff % 32 || c.d_model < 32 || c.d_ff < 32)
        return fail(TSK_ERR_SHAPE, "d_model and d_ff must be multiples of 32 (Q8_0 blocks)");
    if (c.rel_buckets < 2 || c.rel_buckets % 2 || c.rel_max_dist <= c.rel_buckets / 4 || !(c.eps > 0))
        return fail(TSK_ERR_INVALID_ARG, "rel_buckets / rel_max_dist / eps");
    int rc = require_init();
    if (rc) return rc;
    tsk_t5 *t = new tsk_t5();
    t->cfg = c;
    const int L = c.n_layers, d = c.d_model, inner = c.n_heads * c.d_kv, ff = c.d_ff, n = c.max_tokens;
    auto add = [&](const std::string &nm, int64_t a, int64_t b, int type) {
        t->idx[nm] = (int) t->w.size();
        t->w.push_back(T5W{nm, a, b, type});
    };
    add("rel_bias", c.n_heads, c.rel_buckets, TSK_TYPE_F32);
    for (int i = 0; i < L; ++i) {
        const std::string b = "blk." + std::to_string(i);
        add(b + ".attn_norm", d, 1, TSK_TYPE_F32);
        add(b + ".q", d, inner, TSK_TYPE_Q8_0);
        add(b + ".k", d, inner, TSK_TYPE_Q8_0);
        add(b + ".v", d, inner, TSK_TYPE_Q8_0);
        add(b + ".o", inner, d, TSK_TYPE_Q8_0);
        add(b + ".ffn_norm", d, 1, TSK_TYPE_F32);
        add(b + ".wi_0", d, ff, TSK_TYPE_Q8_0);
        add(b + ".wi_1", d, ff, TSK_TYPE_Q8_0);
        add(b + ".wo", ff, d, TSK_TYPE_Q8_0);
    }
    add("out_norm", d, 1, TSK_TYPE_F32);

    // device weights: per layer the stacked QKV, O, interleaved wi, wo planes + norms
    auto al = [](size_t b) { return (b + 255) & ~(size_t) 255; };
    auto planes = [&](int64_t K, int64_t M) { return al((size_t) (K * M)) + al((size_t) (M * (K / 32)) * 2); };
    const size_t per_layer = planes(d, 3 * inner) + planes(inner, d) + planes(d, 2 * ff) + planes(ff, d) + 2 * al(4 * d);
    const size_t total = per_layer * L + al((size_t) 4 * c.n_heads * c.rel_buckets) + al((size_t) 4 * d);
    auto alloc = [&](void **p, size_t bytes) -> int {
        hipError_t e = hipMalloc(p, bytes);
        if (e != hipSuccess) return fail(TSK_ERR_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return TSK_OK;
    };
    const int kmax = std::max(std::max(d, inner), ff);
    if ((rc = alloc((void **) &t->blob, total)) ||
        (rc = alloc((void **) &t->x, sizeof(float) * n * d)) ||
        (rc = alloc((void **) &t->h, sizeof(float) * n * d)) ||
        (rc = alloc((void **) &t->qkv, sizeof(float) * n * 3 * inner)) ||
        (rc = alloc((void **) &t->att, sizeof(float) * n * inner)) ||
        (rc = alloc((void **) &t->g, sizeof(float) * n * ff)) ||
        (rc = alloc((void **) &t->rel_lut, sizeof(float) * c.n_heads * (2 * n - 1))) ||
        (rc = alloc((void **) &t->ones, sizeof(float) * d)) ||
        (rc = alloc((void **) &t->qx, (size_t) n * kmax)) ||
        (rc = alloc((void **) &t->dx, sizeof(float) * n * (kmax / 32))) ||
        (rc = alloc((void **) &t->bkt, sizeof(int32_t) * (2 * n - 1))) ||
        (rc = alloc((void **) &t->valid, n)) ||
        (rc = alloc((void **) &t->io, sizeof(float) * 2 * n * d))) {
        tsk_t5_destroy(t);
        return rc;
    }
    char *p = t->blob;
    auto take = [&](size_t bytes) { char *r = p; p += al(bytes); return r; };
    for (int i = 0; i < L; ++i) {
        Layer ly;
        ly.qkv_q = (int8_t *) take((size_t) d * 3 * inner); ly.qkv_d = (uint16_t *) take((size_t) 3 * inner * (d / 32) * 2);
        ly.o_q = (int8_t *) take((size_t) inner * d); ly.o_d = (uint16_t *) take((size_t) d * (inner / 32) * 2);
        ly.wi_q = (int8_t *) take((size_t) d * 2 * ff); ly.wi_d = (uint16_t *) take((size_t) 2 * ff * (d / 32) * 2);
        ly.wo_q = (int8_t *) take((size_t) ff * d); ly.wo_d = (uint16_t *) take((size_t) d * (ff / 32) * 2);
        ly.attn_norm = (float *) take(4 * d); ly.ffn_norm = (float *) take(4 * d);
        t->layers.push_back(ly);
    }
    t->rel_bias = (float *) take((size_t) 4 * c.n_heads * c.rel_buckets);
    t->out_norm = (float *) take((size_t) 4 * d);
    hipError_t e = hipMemset(t->blob, 0, total);
    if (e == hipSuccess) {
        launch_kernel(fill_kernel, dim3((d + 255) / 256), dim3(256), 0, nullptr, t->ones, (int64_t) d, 1.0f);
        e = hipGetLastError();
    }
    // bucket ids of every relative distance the capacity allows (host, as :95)
    if (e == hipSuccess) {
        std::vector<int32_t> bk(2 * n - 1);
        for (int r = -(n - 1); r <= n - 1; ++r) bk[r + n - 1] = t5_bucket(r, c.rel_buckets, c.rel_max_dist);
        e = hipMemcpy(t->bkt, bk.data(), sizeof(int32_t) * bk.size(), hipMemcpyHostToDevice);
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        tsk_t5_destroy(t);
        return hip_fail(e, "t5 create");
    }
    *out = t;
    return TSK_OK;
}

extern "C" int tsk_t5_n_tensors(const tsk_t5 *t) { return t ? (int) t->w.size() : 0; }

extern "C" int tsk_t5_tensor_info(const tsk_t5 *t, int i, const char **name, int64_t ne[4], int *type) {
    if (!t || i < 0 || i >= (int) t->w.size()) return fail(TSK_ERR_INVALID_ARG, "tensor index %d", i);
    if (name) *name = t->w[i].name.c_str();
    if (ne) { ne[0] = t->w[i].ne0; ne[1] = t->w[i].ne1; ne[2] = 1; ne[3] = 1; }
    if (type) *type = t->w[i].type;
    return TSK_OK;
}

// Q8_0 blocks of a [K][M] weight -> rows (dst_row0 + r * row_step) of the
// int8 / fp16 planes of a stacked [Mtot][K] weight (bit-preserving)
static int put_q8(const void *src, int64_t K, int64_t M, int8_t *qd, uint16_t *dd, int64_t row0, int64_t step) {
    const int64_t KB = K / 32;
    std::vector<int8_t> q((size_t) (K * M));
    std::vector<uint16_t> dv((size_t) (KB * M));
    const uint8_t *b = (const uint8_t *) src;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t kb = 0; kb < KB; ++kb) {
            const uint8_t *blk = b + (m * KB + kb) * 34;
            memcpy(&dv[(size_t) (m * KB + kb)], blk, 2);
            memcpy(&q[(size_t) (m * K + kb * 32)], blk + 2, 32);
        }
    hipError_t e;
    if (step == 1) {
        e = hipMemcpy(qd + row0 * K, q.data(), (size_t) (K * M), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(dd + row0 * KB, dv.data(), (size_t) (KB * M) * 2, hipMemcpyHostToDevice);
    } else {
        e = hipMemcpy2D(qd + row0 * K, (size_t) (step * K), q.data(), (size_t) K, (size_t) K, (size_t) M,
                        hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy2D(dd + row0 * KB, (size_t) (step * KB * 2), dv.data(), (size_t) (KB * 2), (size_t) (KB * 2),
                            (size_t) M, hipMemcpyHostToDevice);
    }
    return hipcheck(e, "t5 weight upload");
}

extern "C" int tsk_t5_set_tensor(tsk_t5 *t, const char *name, const void *src, size_t nbytes) {
    if (!t || !name || !src) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = t->idx.find(name);
    if (it == t->idx.end()) return fail(TSK_ERR_INVALID_ARG, "unknown tensor '%s'", name);
    const T5W &w = t->w[it->second];
    const size_t want = w.type == TSK_TYPE_Q8_0 ? (size_t) (w.ne0 / 32) * 34 * (size_t) w.ne1 : (size_t) (w.ne0 * w.ne1) * 4;
    if (nbytes != want) return fail(TSK_ERR_SHAPE, "'%s' needs %zu bytes, got %zu", name, want, nbytes);
    const tsk_t5_config &c = t->cfg;
    const int64_t inner = (int64_t) c.n_heads * c.d_kv;
    if (w.name == "rel_bias") return hipcheck(hipMemcpy(t->rel_bias, src, nbytes, hipMemcpyHostToDevice), "upload");
    if (w.name == "out_norm") return hipcheck(hipMemcpy(t->out_norm, src, nbytes, hipMemcpyHostToDevice), "upload");
    // blk.<i>.<part>
    const int li = atoi(w.name.c_str() + 4);
    const std::string part = w.name.substr(w.name.find('.', 4) + 1);
    Layer &ly = t->layers[li];
    if (part == "attn_norm") return hipcheck(hipMemcpy(ly.attn_norm, src, nbytes, hipMemcpyHostToDevice), "upload");
    if (part == "ffn_norm") return hipcheck(hipMemcpy(ly.ffn_norm, src, nbytes, hipMemcpyHostToDevice), "upload");
    if (part == "q") return put_q8(src, w.ne0, w.ne1, ly.qkv_q, ly.qkv_d, 0, 1);
    if (part == "k") return put_q8(src, w.ne0, w.ne1, ly.qkv_q, ly.qkv_d, inner, 1);
    if (part == "v") return put_q8(src, w.ne0, w.ne1, ly.qkv_q, ly.qkv_d, 2 * inner, 1);
    if (part == "o") return put_q8(src, w.ne0, w.ne1, ly.o_q, ly.o_d, 0, 1);
    if (part == "wi_0") return put_q8(src, w.ne0, w.ne1, ly.wi_q, ly.wi_d, 0, 2);
    if (part == "wi_1") return put_q8(src, w.ne0, w.ne1, ly.wi_q, ly.wi_d, 1, 2);
    if (part == "wo") return put_q8(src, w.ne0, w.ne1, ly.wo_q, ly.wo_d, 0, 1);
    return fail(TSK_ERR_INVALID_ARG, "tensor '%s'", name);
}

extern "C" int tsk_t5_encode_layers(tsk_t5 *t, int n, const float *x_d, const int32_t *ids, int layer_begin,
                                    int layer_end, int final_norm, float *out_d, tsk_stream stream) {
    if (!t || !x_d || !ids || !out_d) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    const tsk_t5_config &c = t->cfg;
    if (n < 1 || n > c.max_tokens) return fail(TSK_ERR_SHAPE, "n=%d outside [1, %d]", n, c.max_tokens);
    if (layer_begin < 0 || layer_end > c.n_layers || layer_begin > layer_end)
        return fail(TSK_ERR_INVALID_ARG, "layers [%d, %d) outside [0, %d)", layer_begin, layer_end, c.n_layers);
    int rc = require_init();
    if (rc) return rc;
    hipStream_t s = (hipStream_t) stream;
    const int d = c.d_model, H = c.n_heads, inner = H * c.d_kv, ff = c.d_ff;
    // key padding (t5_encoder.cpp:97) and the per-head bias + padding mask
    std::vector<uint8_t> valid(n);
    for (int i = 0; i < n; ++i) valid[i] = ids[i] != 0;
    if ((rc = hipcheck(hipMemcpyAsync(t->valid, valid.data(), n, hipMemcpyHostToDevice, s), "ids"))) return rc;
    if ((rc = hipcheck(hipStreamSynchronize(s), "ids"))) return rc;    // `valid` is a host temporary
    const int64_t nl = (int64_t) H * (2 * c.max_tokens - 1);
    launch_kernel(t5_lut_kernel, dim3((unsigned) ((nl + 255) / 256)), dim3(256), 0, s, (const float *) t->rel_bias,
                  (const int32_t *) t->bkt, H, c.max_tokens, t->rel_lut);
    if ((rc = hipcheck(hipGetLastError(), "t5 bias table"))) return rc;
    if ((rc = hipcheck(hipMemcpyAsync(t->x, x_d, sizeof(float) * n * d, hipMemcpyDeviceToDevice, s), "x"))) return rc;

    // attention over the qkv rows [n][3 * inner] (ggml ne [64, n, H, 1]), F32
    // q / k / v, scale 1, output rows of inner ([64, H, n, 1])
    AttnParams ap;
    memset(&ap, 0, sizeof(ap));
    ap.q = t->qkv; ap.k = t->qkv + inner; ap.v = t->qkv + 2 * inner; ap.o = t->att;
    ap.q_type = ap.kv_type = TSK_TYPE_F32;
    ap.Nq = ap.Nkv = n; ap.H = ap.Hkv = H; ap.B = 1;
    ap.q_nb1 = ap.k_nb1 = ap.v_nb1 = (int64_t) 3 * inner * 4;
    ap.q_nb2 = ap.k_nb2 = ap.v_nb2 = 64 * 4;
    ap.q_nb3 = ap.k_nb3 = ap.v_nb3 = (int64_t) 3 * inner * 4 * n;
    ap.m_ne2 = ap.m_ne3 = 1;
    ap.o_nb1 = 64 * 4; ap.o_nb2 = (int64_t) inner * 4; ap.o_nb3 = (int64_t) inner * 4 * n;
    ap.scale = 1.0f;
    ap.n_head_log2 = 1u << (uint32_t) floorf(log2f((float) H));
    ap.m0 = ap.m1 = 1.0f;
    ap.rel_lut = t->rel_lut; ap.rel_nh = 2 * c.max_tokens - 1; ap.rel_off = c.max_tokens - 1;
    ap.key_valid = t->valid;

    for (int i = layer_begin; i < layer_end; ++i) {
        const Layer &ly = t->layers[i];
        if ((rc = rmsnorm_q8(t, t->x, ly.attn_norm, c.eps, n, d, s))) return rc;
        if ((rc = q8_gemm(t, ly.qkv_q, ly.qkv_d, n, d, 3 * inner, EPI_STORE, t->qkv, 3 * inner, nullptr, s))) return rc;
        if ((rc = hipcheck(launch_attention(ap, s), "t5 attention"))) return rc;
        if ((rc = quantize(t, t->att, n, inner, s))) return rc;
        if ((rc = q8_gemm(t, ly.o_q, ly.o_d, n, inner, d, EPI_GATE_RES, nullptr, 0, t->x, s))) return rc;
        if ((rc = rmsnorm_q8(t, t->x, ly.ffn_norm, c.eps, n, d, s))) return rc;
        if ((rc = q8_gemm(t, ly.wi_q, ly.wi_d, n, d, 2 * ff, EPI_GEGLU, t->g, ff, nullptr, s))) return rc;
        if ((rc = quantize(t, t->g, n, ff, s))) return rc;
        if ((rc = q8_gemm(t, ly.wo_q, ly.wo_d, n, ff, d, EPI_GATE_RES, nullptr, 0, t->x, s))) return rc;
    }
    if (final_norm) return rmsnorm(t->x, t->out_norm, c.eps, n, d, out_d, s);
    return hipcheck(hipMemcpyAsync(out_d, t->x, sizeof(float) * n * d, hipMemcpyDeviceToDevice, s), "out copy");
}

extern "C" int tsk_t5_encode_device(tsk_t5 *t, int n, const float *x_d, const int32_t *ids, float *out_d,
                                    tsk_stream stream) {
    if (!t) return fail(TSK_ERR_INVALID_ARG, "t5 is NULL");
    return tsk_t5_encode_layers(t, n, x_d, ids, 0, t->cfg.n_layers, 1, out_d, stream);
}

extern "C" int tsk_t5_encode(tsk_t5 *t, int n, const float *x, const int32_t *ids, float *out, tsk_stream stream) {
    if (!t) return fail(TSK_ERR_INVALID_ARG, "t5 is NULL");
    return tsk_t5_encode_range(t, n, x, ids, 0, t->cfg.n_layers, 1, out, stream);
}

extern "C" int tsk_t5_encode_range(tsk_t5 *t, int n, const float *x, const int32_t *ids, int layer_begin,
                                   int layer_end, int final_norm, float *out, tsk_stream stream) {
    if (!t || !x || !ids || !out) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    if (n < 1 || n > t->cfg.max_tokens) return fail(TSK_ERR_SHAPE, "n=%d outside [1, %d]", n, t->cfg.max_tokens);
    hipStream_t s = (hipStream_t) stream;
    const size_t bytes = sizeof(float) * n * t->cfg.d_model;
    float *xin = t->io, *xo = t->io + (size_t) n * t->cfg.d_model;
    int rc = hipcheck(hipMemcpyAsync(xin, x, bytes, hipMemcpyHostToDevice, s), "x upload");
    if (!rc) rc = tsk_t5_encode_layers(t, n, xin, ids, layer_begin, layer_end, final_norm, xo, stream);
    if (!rc) rc = hipcheck(hipMemcpyAsync(out, xo, bytes, hipMemcpyDeviceToHost, s), "out download");
    // on every path: the caller's host buffers are done with once the stream is
    const hipError_t e = hipStreamSynchronize(s);
    if (!rc) rc = hipcheck(e, "sync");
    return rc;
}
