// vae.cpp — the Oobleck VAE decoder of ts_vae::decode (src/vae_decoder.cpp:
// 62-124) on gfx950, F32 throughout (the converter keeps the VAE F32).
//
// Activations are token-major rows [T][C] (channels fastest), so every
// convolution is one F32 GEMM over implicit im2col rows (launch_gemm_f32,
// fp32 MFMA): y[t][oc] = sum_{kw, ic} W[oc][kw][ic] x[t + kw d - p][ic].
// The reference keeps [T, C] with time fastest and runs im2col + mul_mat; the
// sums are the same products in another order.
//
// Transposed convolution (stride s, kernel K = 2 s, padding s / 2): the
// reference zero-stuffs the input (s - 1 zeros after every frame) and runs a
// stride-1 conv1d with the converter's flipped kernel W' and padding
// K - 1 - s / 2 (:36-58). Output t = s q + r then takes exactly two taps,
// k = k0(r) and k0(r) + s with k0(r) = (K - 1 - s / 2 - r) mod s, reading
// input frames q + c(r) and q + c(r) + 1, c(r) = (r + k0(r) - (K - 1 - s / 2)) / s
// in {-1, 0}. All s phases read frames q - 1, q, q + 1: one 3-tap convolution
// (padding 1) with s * OC output channels -- channel r * OC + oc holds phase r
// -- whose output rows [T][s * OC] are the upsampled rows [s T][OC]. Each
// phase's unused tap is a zero weight, so every output is the reference's
// sum of the same two products (plus zero terms, which change no fp32 sum).
// The phases with c(r) = -1 come first (r < s / 2 for K = 2 s), so the merged
// kernel runs as two 2-tap products over those two channel ranges (taps 0, 1
// with padding 1; taps 1, 2 without), skipping the zero taps.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/tsk/tsk.h"
#include "host_convert.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

using namespace tsk;

namespace {

struct VW {
    std::string name;
    int64_t ne[3];
    bool conv, ct;          // convolution kernel; transposed-convolution kernel
    int stride;             // ct: the stride s
    size_t offset;          // device float offset of the prepared layout
    size_t count;           // floats stored
    size_t offset16;        // split products: bf16 offset of the planes (3 count: [hi | lo | hi] per IC group)
};

}  // namespace

struct tsk_vae {
    tsk_vae_config cfg;
    std::vector<VW> w;
    std::unordered_map<std::string, int> idx;
    float *blob = nullptr;
    float *act[3] = {nullptr, nullptr, nullptr};   // activation rows, max_latent * hop * channels each
    float *lat = nullptr;                          // latent rows [T][latent_dim]
    size_t act_cap = 0;
    int hop = 1;
    // F32 products as three bf16 ones (opt-in, TSK_VAE_SPLIT=1 when the model
    // is created; every channel count a multiple of 64): the kernels' split
    // planes, and the activations the convolutions read as split planes
    // [T][3 C] (two buffers and the latent)
    bool split = false;
    uint16_t *blob16 = nullptr;
    uint16_t *ap[2] = {nullptr, nullptr};
    uint16_t *latp = nullptr;
};

namespace {

int hipcheck(hipError_t e, const char *what) { return e == hipSuccess ? TSK_OK : hip_fail(e, what); }

void addv(tsk_vae *v, const std::string &name, int64_t a, int64_t b, int64_t c, bool conv, bool ct = false,
          int stride = 0) {
    VW x;
    x.name = name;
    x.ne[0] = a; x.ne[1] = b; x.ne[2] = c;
    x.conv = conv;
    x.ct = ct;
    x.stride = stride;
    x.offset = x.offset16 = 0;
    // prepared layouts: conv kw-major [OC][K * IC]; transposed conv the merged
    // 3-tap kernel [s * OC][3 * IC] and its bias replicated [s * OC]
    x.count = ct ? (size_t) stride * c * 3 * b : (size_t) (a * b * c);
    v->idx[name] = (int) v->w.size();
    v->w.push_back(x);
}

// channels of decoder block n (n = 0 .. 4 -> decoder.layers.1 .. 5): in, out, stride
void block_dims(const tsk_vae_config &c, int n, int *in, int *out, int *s) {
    const int mult[6] = {1, c.c_mults[0], c.c_mults[1], c.c_mults[2], c.c_mults[3], c.c_mults[4]};
    *in = mult[5 - n] * c.channels;
    *out = mult[4 - n] * c.channels;
    *s = c.strides[4 - n];
}

const VW &wi(const tsk_vae *v, const std::string &n) { return v->w[v->idx.at(n)]; }
const float *wp(const tsk_vae *v, const std::string &n) { return v->blob + wi(v, n).offset; }

// the SnakeBeta of the named parameters over C channels, for a GEMM epilogue:
// in place of the output (y2 null) or next to it into y2
F32Snake snake_epi(const tsk_vae *v, const std::string &p, int C, float *y2) {
    return F32Snake{wp(v, p + ".alpha"), wp(v, p + ".beta"), y2, C};
}

// y rows [T_out][OC] = conv(x rows [T_in][IC]) + bias, stride 1 (F32 GEMM),
// optionally followed by a SnakeBeta
int conv(const tsk_vae *v, const std::string &p, bool bias, const float *x, int IC, int T_in, int pad, int dil,
         float *y, bool accumulate, hipStream_t s, const F32Snake *sk = nullptr) {
    const VW &w = wi(v, p + ".weight");
    const int KW = (int) w.ne[0], OC = (int) w.ne[2];
    GemmProblem q;
    memset(&q, 0, sizeof(q));
    q.x = x; q.ld_x = IC;
    q.wf = wp(v, p + ".weight"); q.ld_w = (int64_t) KW * IC;
    q.bias = bias ? wp(v, p + ".bias") : nullptr;
    q.y = y; q.ld_y = OC;
    const int T_out = T_in + 2 * pad - dil * (KW - 1);
    q.M = OC; q.N = T_out; q.K = KW * IC; q.splits = 1;
    if (KW > 1 || pad) {
        q.conv_ic = IC; q.conv_iw = T_in; q.conv_ow = T_out; q.conv_s = 1; q.conv_p = pad; q.conv_d = dil;
    }
    q.accumulate = accumulate ? 1 : 0;
    return hipcheck(launch_gemm_f32(q, 0, s, sk), "vae conv");
}

// the first phase that reads input frames q and q + 1 (c(r) = 0) when the
// phases r < it all read q - 1 and q (c(r) = -1), else -1
int ct_split_phase(int64_t K, int64_t st) {
    const int64_t P = K - 1 - st / 2;
    int first0 = -1;
    for (int64_t r = 0; r < st; ++r) {
        const int64_t k0 = ((P - r) % st + st) % st, c0 = (r + k0 - P) / st;
        if (c0 == 0 && first0 < 0) first0 = (int) r;
        if (c0 == -1 && first0 >= 0) return -1;
    }
    return first0 < 0 ? (int) st : first0;
}

// transposed convolution as the merged 3-tap convolution: y rows [s T_in][OC].
// Each phase uses two of the three taps, so it runs as two 2-tap products:
// the phases reading frames q - 1, q (taps 0, 1, padding 1) and those
// reading q, q + 1 (taps 1, 2, no padding), a third fewer products than the
// 3-tap kernel whose zero taps added nothing to any sum.
int conv_t(const tsk_vae *v, const std::string &p, const float *x, int IC, int T_in, float *y, hipStream_t s,
           const F32Snake *sk = nullptr) {
    const VW &w = wi(v, p + ".weight");
    const int OC = (int) w.ne[2], st = w.stride;
    const float *wf = wp(v, p + ".weight"), *bias = wp(v, p + ".bias");
    const int ra = ct_split_phase(w.ne[0], st);
    GemmProblem q;
    memset(&q, 0, sizeof(q));
    q.x = x; q.ld_x = IC;
    q.ld_w = (int64_t) 3 * IC;
    q.ld_y = (int64_t) st * OC;
    q.N = T_in; q.splits = 1;
    q.conv_ic = IC; q.conv_iw = T_in; q.conv_ow = T_in; q.conv_s = 1; q.conv_d = 1;
    if (ra < 0) {
        q.wf = wf; q.bias = bias; q.y = y;
        q.M = st * OC; q.K = 3 * IC; q.conv_p = 1;
        return hipcheck(launch_gemm_f32(q, 0, s, sk), "vae transposed conv");
    }
    for (int g = 0; g < 2; ++g) {
        const int r0 = g ? ra : 0, r1 = g ? st : ra;
        if (r1 <= r0) continue;
        const int64_t row0 = (int64_t) r0 * OC;
        q.wf = wf + row0 * 3 * IC + (g ? IC : 0);      // taps 1, 2 for the second group
        q.bias = bias + row0;
        q.y = y + row0;
        q.M = (r1 - r0) * OC; q.K = 2 * IC; q.conv_p = g ? 0 : 1;
        F32Snake sg;
        if (sk) {
            sg = *sk;                                   // row0 is a multiple of the period OC
            if (sg.y2) sg.y2 += row0;
        }
        const int rc = hipcheck(launch_gemm_f32(q, 0, s, sk ? &sg : nullptr), "vae transposed conv");
        if (rc) return rc;
    }
    return TSK_OK;
}

// ---- split products: the cooperative bf16 GEMM over 3 IC (weight planes
// [hi | lo | hi] against input planes [hi | hi | lo]: x w up to x_lo w_lo and
// the lo roundings, ~2^-17 of |x w| per term) with the EPI_F32X epilogue:
// bias, the residual update, and the SnakeBeta `snake` (parameters of
// period C) into the split planes yp the next convolution reads, or into an
// f32 y2 (the final snake, for the fp32 output convolution)
struct SplitOut {
    float *y;           // f32 output rows (nullable: not written)
    bool accumulate;    // y += conv
    const char *snake;  // SnakeBeta parameters' prefix, or null
    int C;              // its period (channels)
    float *y2;          // the snake as f32 rows
    uint16_t *yp;       // the snake as split planes
};

void set_out(const tsk_vae *v, GemmProblem &q, const SplitOut &o) {
    q.y = o.y;
    q.accumulate = o.accumulate ? 1 : 0;
    if (o.snake) {
        q.snk_ea = wp(v, std::string(o.snake) + ".alpha");
        q.snk_eb = wp(v, std::string(o.snake) + ".beta");
        q.snk_period = o.C;
        q.y2 = o.y2;
        q.yp = o.yp;
    }
}

int conv_split(const tsk_vae *v, const std::string &p, const uint16_t *xp, int IC, int T_in, int pad, int dil,
               const SplitOut &o, hipStream_t s) {
    const VW &w = wi(v, p + ".weight");
    const int KW = (int) w.ne[0], OC = (int) w.ne[2];
    GemmGroup g;
    memset(&g, 0, sizeof(g));
    g.nprob = 1;
    GemmProblem &q = g.p[0];
    q.x = xp; q.ld_x = 3 * IC;
    q.w = v->blob16 + w.offset16; q.ld_w = (int64_t) KW * 3 * IC;
    q.bias = wp(v, p + ".bias");
    q.ld_y = OC;
    const int T_out = T_in + 2 * pad - dil * (KW - 1);
    q.M = OC; q.N = T_out; q.K = KW * 3 * IC; q.splits = 1;
    if (KW > 1 || pad) {
        q.conv_ic = 3 * IC; q.conv_iw = T_in; q.conv_ow = T_out; q.conv_s = 1; q.conv_p = pad; q.conv_d = dil;
    }
    set_out(v, q, o);
    return hipcheck(launch_gemm_coop(g, EPI_F32X, s), "vae split conv");
}

// the transposed convolution of conv_t over the split planes: the merged
// kernel's planes [s OC][3 taps][3 IC], its two-tap phase groups
int conv_t_split(const tsk_vae *v, const std::string &p, const uint16_t *xp, int IC, int T_in, const SplitOut &o,
                 hipStream_t s) {
    const VW &w = wi(v, p + ".weight");
    const int OC = (int) w.ne[2], st = w.stride;
    const uint16_t *wq = v->blob16 + w.offset16;
    const float *bias = wp(v, p + ".bias");
    const int ra = ct_split_phase(w.ne[0], st);
    GemmGroup g;
    memset(&g, 0, sizeof(g));
    g.nprob = 1;
    GemmProblem &q = g.p[0];
    q.x = xp; q.ld_x = 3 * IC;
    q.ld_w = (int64_t) 9 * IC;
    q.ld_y = (int64_t) st * OC;
    q.N = T_in; q.splits = 1;
    q.conv_ic = 3 * IC; q.conv_iw = T_in; q.conv_ow = T_in; q.conv_s = 1; q.conv_d = 1;
    set_out(v, q, o);
    if (ra < 0) {
        q.w = wq; q.bias = bias;
        q.M = st * OC; q.K = 9 * IC; q.conv_p = 1;
        return hipcheck(launch_gemm_coop(g, EPI_F32X, s), "vae split transposed conv");
    }
    for (int gi = 0; gi < 2; ++gi) {
        const int r0 = gi ? ra : 0, r1 = gi ? st : ra;
        if (r1 <= r0) continue;
        const int64_t row0 = (int64_t) r0 * OC;
        q.w = wq + row0 * 9 * IC + (gi ? 3 * IC : 0);   // taps 1, 2 for the second group
        q.bias = bias + row0;
        q.y = o.y ? o.y + row0 : nullptr;
        q.y2 = o.y2 ? o.y2 + row0 : nullptr;
        q.yp = o.yp ? o.yp + 3 * row0 : nullptr;          // row0 is a multiple of the period OC
        q.M = (r1 - r0) * OC; q.K = 6 * IC; q.conv_p = gi ? 0 : 1;
        const int rc = hipcheck(launch_gemm_coop(g, EPI_F32X, s), "vae split transposed conv");
        if (rc) return rc;
    }
    return TSK_OK;
}

int validate(const tsk_vae_config *c) {
    if (!c) return fail(TSK_ERR_INVALID_ARG, "cfg is NULL");
    if (c->latent_dim < 4 || c->latent_dim % 4 || c->channels < 4 || c->channels % 4 || c->out_channels < 1 ||
        c->max_latent < 1)
        return fail(TSK_ERR_SHAPE, "latent_dim and channels must be multiples of 4");
    int64_t hop = 1;
    for (int i = 0; i < 5; ++i) {
        if (c->c_mults[i] < 1 || c->strides[i] < 2 || c->strides[i] % 2)
            return fail(TSK_ERR_SHAPE, "c_mults >= 1, strides even");
        hop *= c->strides[i];
    }
    if ((int64_t) c->max_latent * hop > (1 << 28)) return fail(TSK_ERR_SHAPE, "max_latent * hop too large");
    return TSK_OK;
}

}  // namespace

extern "C" void tsk_vae_default_config(tsk_vae_config *c) {
    if (!c) return;
    c->latent_dim = 64; c->channels = 128; c->out_channels = 2;
    const int m[5] = {1, 2, 4, 8, 16}, st[5] = {2, 4, 4, 8, 8};
    for (int i = 0; i < 5; ++i) { c->c_mults[i] = m[i]; c->strides[i] = st[i]; }
    c->max_latent = 646;
}

extern "C" void tsk_vae_destroy(tsk_vae *v) {
    if (!v) return;
    (void) hipDeviceSynchronize();
    if (v->blob) (void) hipFree(v->blob);
    for (float *a : v->act)
        if (a) (void) hipFree(a);
    if (v->lat) (void) hipFree(v->lat);
    if (v->blob16) (void) hipFree(v->blob16);
    for (uint16_t *a : v->ap)
        if (a) (void) hipFree(a);
    if (v->latp) (void) hipFree(v->latp);
    delete v;
}

extern "C" int tsk_vae_create(const tsk_vae_config *cfg, tsk_vae **out) {
    if (!out) return fail(TSK_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    int rc = validate(cfg);
    if (rc) return rc;
    if ((rc = require_init())) return rc;
    tsk_vae *v = new tsk_vae();
    v->cfg = *cfg;
    const tsk_vae_config &c = v->cfg;
    int in0, out0, s0;
    block_dims(c, 0, &in0, &out0, &s0);
    // the converter's names (convert/convert_vae.py:34-56, src/vae_decoder.cpp:73-107)
    addv(v, "decoder.layers.0.weight", 7, c.latent_dim, in0, true);
    addv(v, "decoder.layers.0.bias", in0, 1, 1, false);
    int64_t max_ch_t = (int64_t) in0;                 // largest channels x frames per latent frame
    int64_t up = 1;
    for (int n = 0; n < 5; ++n) {
        int ci, co, st;
        block_dims(c, n, &ci, &co, &st);
        const std::string bp = "decoder.layers." + std::to_string(n + 1);
        addv(v, bp + ".layers.0.alpha", ci, 1, 1, false);
        addv(v, bp + ".layers.0.beta", ci, 1, 1, false);
        addv(v, bp + ".layers.1.weight", 2 * st, ci, co, true, true, st);
        addv(v, bp + ".layers.1.bias", co, 1, 1, false, false, st);   // replicated over the s phases
        v->w.back().count = (size_t) st * co;
        for (int r = 0; r < 3; ++r) {
            const std::string rp = bp + ".layers." + std::to_string(r + 2);
            addv(v, rp + ".layers.0.alpha", co, 1, 1, false);
            addv(v, rp + ".layers.0.beta", co, 1, 1, false);
            addv(v, rp + ".layers.1.weight", 7, co, co, true);
            addv(v, rp + ".layers.1.bias", co, 1, 1, false);
            addv(v, rp + ".layers.2.alpha", co, 1, 1, false);
            addv(v, rp + ".layers.2.beta", co, 1, 1, false);
            addv(v, rp + ".layers.3.weight", 1, co, co, true);
            addv(v, rp + ".layers.3.bias", co, 1, 1, false);
        }
        up *= st;
        max_ch_t = std::max(max_ch_t, up * co);
    }
    int lin, lout, ls;
    block_dims(c, 4, &lin, &lout, &ls);
    addv(v, "decoder.layers.6.alpha", lout, 1, 1, false);
    addv(v, "decoder.layers.6.beta", lout, 1, 1, false);
    addv(v, "decoder.layers.7.weight", 7, lout, c.out_channels, true);
    v->hop = (int) up;
    max_ch_t = std::max(max_ch_t, up * c.out_channels);
    size_t off = 0;
    for (auto &x : v->w) {
        x.offset = off;
        off += (x.count + 63) & ~(size_t) 63;
    }
    v->act_cap = (size_t) c.max_latent * (size_t) max_ch_t;
    // split products (opt-in) when every convolution's channels fit the
    // cooperative bf16 GEMM's 64-wide stages over 3 IC (the final k7 stays
    // fp32 products). The decoder amplifies a product's relative error about
    // 50-100 times on its way to the audio: split products (~2^-17 per term)
    // leave the audio ~5e-4 rel-L2 from fp32 products (fp32 ones: ~6e-5 from
    // an fp64 decode), 1.6-1.7 times faster
    v->split = tuning().vae_split && c.latent_dim % 64 == 0;
    for (int n = 0; n < 5; ++n) {
        int ci, co, st;
        block_dims(c, n, &ci, &co, &st);
        v->split = v->split && ci % 64 == 0 && co % 64 == 0;
    }
    size_t off16 = 0;
    if (v->split)
        for (auto &x : v->w)
            if ((x.conv || x.ct) && x.name != "decoder.layers.7.weight") {
                x.offset16 = off16;
                off16 += (3 * x.count + 127) & ~(size_t) 127;
            }
    auto alloc = [&](void **p, size_t bytes) -> int {
        hipError_t e = hipMalloc(p, bytes);
        if (e != hipSuccess) return fail(TSK_ERR_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return TSK_OK;
    };
    if ((rc = alloc((void **) &v->blob, sizeof(float) * off)) ||
        (rc = alloc((void **) &v->act[0], sizeof(float) * v->act_cap)) ||
        (rc = alloc((void **) &v->act[1], sizeof(float) * v->act_cap)) ||
        (rc = alloc((void **) &v->act[2], sizeof(float) * v->act_cap)) ||
        (rc = alloc((void **) &v->lat, sizeof(float) * (size_t) c.max_latent * c.latent_dim)) ||
        (v->split && ((rc = alloc((void **) &v->blob16, 2 * off16)) ||
                      (rc = alloc((void **) &v->ap[0], 6 * v->act_cap)) ||
                      (rc = alloc((void **) &v->ap[1], 6 * v->act_cap)) ||
                      (rc = alloc((void **) &v->latp, 6 * (size_t) c.max_latent * c.latent_dim))))) {
        tsk_vae_destroy(v);
        return rc;
    }
    hipError_t e = hipMemset(v->blob, 0, sizeof(float) * off);
    if (e != hipSuccess) { tsk_vae_destroy(v); return hip_fail(e, "vae init"); }
    *out = v;
    return TSK_OK;
}

extern "C" int tsk_vae_n_tensors(const tsk_vae *v) { return v ? (int) v->w.size() : 0; }

extern "C" int tsk_vae_tensor_info(const tsk_vae *v, int i, const char **name, int64_t ne[4]) {
    if (!v || i < 0 || i >= (int) v->w.size()) return fail(TSK_ERR_INVALID_ARG, "tensor index %d", i);
    if (name) *name = v->w[i].name.c_str();
    if (ne) { ne[0] = v->w[i].ne[0]; ne[1] = v->w[i].ne[1]; ne[2] = v->w[i].ne[2]; ne[3] = 1; }
    return TSK_OK;
}

extern "C" int tsk_vae_hop(const tsk_vae *v) { return v ? v->hop : 0; }

// host f32 in ggml / PyTorch order: conv kernels [OC][IC][K]; alpha / beta
// stored as exp(alpha) / exp(-beta) (the snake's two exponentials, :18-19)
extern "C" int tsk_vae_set_tensor(tsk_vae *v, const char *name, const float *src, int64_t n) {
    if (!v || !name || !src) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = v->idx.find(name);
    if (it == v->idx.end()) return fail(TSK_ERR_INVALID_ARG, "unknown tensor '%s'", name);
    const VW &x = v->w[it->second];
    const int64_t N = x.ne[0] * x.ne[1] * x.ne[2];
    if (n != N) return fail(TSK_ERR_SHAPE, "'%s' has %lld elements, got %lld", name, (long long) N, (long long) n);
    std::vector<float> t(x.count, 0.0f);
    const std::string nm = name;
    const bool is_alpha = nm.size() > 6 && nm.compare(nm.size() - 6, 6, ".alpha") == 0;
    const bool is_beta = nm.size() > 5 && nm.compare(nm.size() - 5, 5, ".beta") == 0;
    if (x.ct) {
        // merged 3-tap kernel: row r * OC + oc, tap j (input frame q - 1 + j),
        // channel ic = W'[oc][ic][k] for the phase's two taps k
        const int64_t K = x.ne[0], IC = x.ne[1], OC = x.ne[2], st = x.stride, P = K - 1 - st / 2;
        for (int64_t r = 0; r < st; ++r) {
            const int64_t k0 = ((P - r) % st + st) % st;
            const int64_t c0 = (r + k0 - P) / st;          // -1 or 0 (r + k0 - P is a multiple of st)
            for (int m = 0; m < 2; ++m) {
                const int64_t k = k0 + m * st, j = c0 + m + 1;
                for (int64_t oc = 0; oc < OC; ++oc)
                    for (int64_t ic = 0; ic < IC; ++ic)
                        t[(size_t) (((r * OC + oc) * 3 + j) * IC + ic)] = src[(oc * IC + ic) * K + k];
            }
        }
    } else if (x.conv) {
        const int64_t K = x.ne[0], IC = x.ne[1], OC = x.ne[2];
        for (int64_t oc = 0; oc < OC; ++oc)
            for (int64_t ic = 0; ic < IC; ++ic)
                for (int64_t k = 0; k < K; ++k) t[(size_t) ((oc * K + k) * IC + ic)] = src[(oc * IC + ic) * K + k];
    } else if (x.stride) {
        for (int64_t r = 0; r < x.stride; ++r)
            for (int64_t i = 0; i < n; ++i) t[(size_t) (r * n + i)] = src[i];
    } else {
        for (int64_t i = 0; i < n; ++i) t[i] = is_alpha ? expf(src[i]) : is_beta ? expf(-src[i]) : src[i];
    }
    hipError_t e = hipMemcpy(v->blob + x.offset, t.data(), sizeof(float) * t.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && v->split && (x.conv || x.ct) && x.name != "decoder.layers.7.weight") {
        // the prepared rows in groups of IC -> [hi | lo | hi] per group,
        // hi = bf16(w), lo = bf16(w - hi)
        const size_t G = (size_t) x.ne[1];
        std::vector<uint16_t> sp(3 * x.count);
        for (size_t g0 = 0; g0 < x.count; g0 += G)
            for (size_t i = 0; i < G; ++i) {
                const float w = t[g0 + i];
                const uint16_t hi = host_bf16_bits(w);
                const uint32_t hb = (uint32_t) hi << 16;
                float hf;
                memcpy(&hf, &hb, 4);
                uint16_t *d = &sp[3 * g0 + i];
                d[0] = hi;
                d[G] = std::isfinite(hf) ? host_bf16_bits(w - hf) : (uint16_t) 0;
                d[2 * G] = hi;
            }
        e = hipMemcpy(v->blob16 + x.offset16, sp.data(), 2 * sp.size(), hipMemcpyHostToDevice);
    }
    return hipcheck(e, "vae set_tensor copy");
}

namespace {

int decode_impl(tsk_vae *v, int T, const float *latent_d, float *audio_d, hipStream_t st) {
    const tsk_vae_config &c = v->cfg;
    int rc;
    // latent ne = [T, latent_dim] (time fastest) -> rows [T][latent_dim]
    if ((rc = hipcheck(launch_transpose_ct(latent_d, 1, c.latent_dim, T, v->lat, st), "vae latent"))) return rc;
    // Every SnakeBeta runs in the epilogue of the convolution that produces
    // its input: x (buffer 0) holds the residual stream, sx (buffer 1 or 2)
    // the snake of x that the next convolution reads, t the other one. A
    // convolution never writes the buffer it reads.
    float *x = v->act[0], *sx = v->act[1], *t = v->act[2];
    int in0, out0, s0;
    block_dims(c, 0, &in0, &out0, &s0);
    if (v->split && tuning().vae_split) {
        // the same chain on split products: each snake written as the split
        // planes the next convolution reads (sp, then tp), the residual
        // stream x f32, the final snake f32 (sx) for the output convolution
        uint16_t *sp = v->ap[0], *tp = v->ap[1];
        if ((rc = hipcheck(launch_cast_rows_split3(v->lat, c.latent_dim, 0, T, T, c.latent_dim, v->latp, st),
                           "vae latent planes")) ||
            (rc = conv_split(v, "decoder.layers.0", v->latp, c.latent_dim, T, 3, 1,
                             SplitOut{nullptr, false, "decoder.layers.1.layers.0", in0, nullptr, sp}, st)))
            return rc;
        int64_t fr = T;
        int Cs = in0;
        const int dl[3] = {1, 3, 9};
        for (int n = 0; n < 5; ++n) {
            int ci, co, s;
            block_dims(c, n, &ci, &co, &s);
            const std::string bp = "decoder.layers." + std::to_string(n + 1);
            const std::string sn0 = bp + ".layers.2.layers.0";
            if ((rc = conv_t_split(v, bp + ".layers.1", sp, ci, (int) fr,
                                   SplitOut{x, false, sn0.c_str(), co, nullptr, tp}, st)))
                return rc;
            std::swap(sp, tp);
            fr *= s;
            Cs = co;
            for (int r = 0; r < 3; ++r) {
                const std::string rp = bp + ".layers." + std::to_string(r + 2), sn = rp + ".layers.2";
                if ((rc = conv_split(v, rp + ".layers.1", sp, Cs, (int) fr, 3 * dl[r], dl[r],
                                     SplitOut{nullptr, false, sn.c_str(), Cs, nullptr, tp}, st)))
                    return rc;
                const bool last = n == 4 && r == 2;
                const std::string np = r < 2 ? bp + ".layers." + std::to_string(r + 3) + ".layers.0"
                                     : n < 4 ? "decoder.layers." + std::to_string(n + 2) + ".layers.0"
                                             : std::string("decoder.layers.6");
                if ((rc = conv_split(v, rp + ".layers.3", tp, Cs, (int) fr, 0, 1,
                                     SplitOut{x, true, np.c_str(), Cs, last ? sx : nullptr, last ? nullptr : sp}, st)))
                    return rc;
            }
        }
        const VW &wf7 = wi(v, "decoder.layers.7.weight");
        if (Cs == 128 && wf7.ne[0] == 7 && c.out_channels == 2)
            return hipcheck(launch_conv_small_oc(sx, (int) fr, Cs, 7, 2, wp(v, "decoder.layers.7.weight"), nullptr, 3,
                                                 audio_d, fr, st),
                            "vae final convolution");
        if ((rc = conv(v, "decoder.layers.7", false, sx, Cs, (int) fr, 3, 1, t, false, st))) return rc;
        return hipcheck(launch_transpose_ct(t, 1, (int) fr, c.out_channels, audio_d, st), "vae audio");
    }
    // conv k7 -> snake of block 1 (the conv's own output is not used again)
    F32Snake sk = snake_epi(v, "decoder.layers.1.layers.0", in0, nullptr);
    if ((rc = conv(v, "decoder.layers.0", true, v->lat, c.latent_dim, T, 3, 1, sx, false, st, &sk))) return rc;
    int64_t frames = T;
    int C = in0;
    const int dil[3] = {1, 3, 9};
    for (int n = 0; n < 5; ++n) {
        int ci, co, s;
        block_dims(c, n, &ci, &co, &s);
        const std::string bp = "decoder.layers." + std::to_string(n + 1);
        // x = conv_t(snake(x)); t = snake of the first residual unit's input
        sk = snake_epi(v, bp + ".layers.2.layers.0", co, t);
        if ((rc = conv_t(v, bp + ".layers.1", sx, ci, (int) frames, x, st, &sk))) return rc;
        std::swap(sx, t);
        frames *= s;
        C = co;
        for (int r = 0; r < 3; ++r) {
            // x += conv_k1(snake(conv_k7_dil(snake(x))))  (the residual unit, :99-105)
            const std::string rp = bp + ".layers." + std::to_string(r + 2);
            sk = snake_epi(v, rp + ".layers.2", C, nullptr);
            if ((rc = conv(v, rp + ".layers.1", true, sx, C, (int) frames, 3 * dil[r], dil[r], t, false, st, &sk)))
                return rc;
            // the next snake of x: the next unit's, the next block's, or the final one
            const std::string np = r < 2 ? bp + ".layers." + std::to_string(r + 3) + ".layers.0"
                                 : n < 4 ? "decoder.layers." + std::to_string(n + 2) + ".layers.0"
                                         : std::string("decoder.layers.6");
            sk = snake_epi(v, np, C, sx);
            if ((rc = conv(v, rp + ".layers.3", true, t, C, (int) frames, 0, 1, x, true, st, &sk))) return rc;
        }
    }
    // conv k7 (no bias) of the final snake -> planar audio [out_channels][T_audio]:
    // the stream-per-wave kernel for 128 -> 2 channels, else the GEMM's rows
    // [T_audio][out_channels] and a transpose
    const VW &wf = wi(v, "decoder.layers.7.weight");
    if (C == 128 && wf.ne[0] == 7 && c.out_channels == 2)
        return hipcheck(launch_conv_small_oc(sx, (int) frames, C, 7, 2, wp(v, "decoder.layers.7.weight"), nullptr, 3,
                                             audio_d, frames, st),
                        "vae final convolution");
    if ((rc = conv(v, "decoder.layers.7", false, sx, C, (int) frames, 3, 1, t, false, st))) return rc;
    return hipcheck(launch_transpose_ct(t, 1, (int) frames, c.out_channels, audio_d, st), "vae audio");
}

}  // namespace

extern "C" int tsk_vae_decode_device(tsk_vae *v, int T, const float *latent_d, float *audio_d, tsk_stream stream) {
    if (!v || !latent_d || !audio_d) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    if (T < 1 || T > v->cfg.max_latent) return fail(TSK_ERR_SHAPE, "T=%d outside [1, %d]", T, v->cfg.max_latent);
    int rc = require_init();
    if (rc) return rc;
    return decode_impl(v, T, latent_d, audio_d, (hipStream_t) stream);
}

extern "C" int tsk_vae_decode(tsk_vae *v, int T, const float *latent, float *audio, int64_t *t_audio,
                              tsk_stream stream) {
    if (!v || !latent || !audio) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    if (T < 1 || T > v->cfg.max_latent) return fail(TSK_ERR_SHAPE, "T=%d outside [1, %d]", T, v->cfg.max_latent);
    int rc = require_init();
    if (rc) return rc;
    const tsk_vae_config &c = v->cfg;
    const size_t n_in = (size_t) T * c.latent_dim, n_out = (size_t) T * v->hop * c.out_channels;
    hipStream_t st = (hipStream_t) stream;
    // device staging: the latent at the end of buffer 2 (read by the first
    // transpose, before any convolution writes there), the audio in buffer 0
    // (the residual stream, last read by the last residual unit)
    float *d_lat = v->act[2] + (v->act_cap - n_in);
    float *d_audio = v->act[0];
    if (n_out > v->act_cap) return fail(TSK_ERR_SHAPE, "audio exceeds the capacity");
    if ((rc = hipcheck(hipMemcpyAsync(d_lat, latent, sizeof(float) * n_in, hipMemcpyHostToDevice, st), "latent")))
        return rc;
    if ((rc = decode_impl(v, T, d_lat, d_audio, st))) return rc;
    if ((rc = hipcheck(hipMemcpyAsync(audio, d_audio, sizeof(float) * n_out, hipMemcpyDeviceToHost, st), "audio")))
        return rc;
    if ((rc = hipcheck(hipStreamSynchronize(st), "sync"))) return rc;
    if (t_audio) *t_audio = (int64_t) T * v->hop;
    return TSK_OK;
}
