// mmdit_graph.cpp — the reference's MM-DiT graph on gfx950: ts_dit::load,
// ts_dit::forward and ts_dit::sample as src/mmdit.cpp:104-376 build them
// (counterpart of src/mmdit.h:9-42), with the kernels of this library:
//   audio_input_proj: conv k3 -> silu -> convMLP                 (:150-155)
//   t_embed MLP                                                   (:157-161)
//   clip_input_proj: linear -> silu -> convMLP                    (:165-167)
//   sync + pos_emb -> conv k7 -> silu -> convMLP -> nearest-exact (:168-178)
//   text: pad text_f, concat t5 -> linear -> silu -> MLP          (:179-183)
//   global_c = t_emb + global_cond_mlp(clip_cond(mean clip) + text_cond(g))
//   extended_c = sync + global_c                                  (:184-196)
//   7 joint blocks over latent | clip | text (the last clip / text pre_only),
//   14 fused blocks on the latent, all with conv k3 linear1 / convMLP on the
//   latent and clip streams and linear / MLP on text              (:203-281)
//   final adaLN(extended_c) -> LN / modulate -> conv k7           (:284-289)
//
// Weights are held in the type the model file gives each tensor, and every
// product follows ggml_mul_mat's semantics for that type (src1 converted to
// the weight's vec_dot type): BF16 (the input rounded to bf16, fp32 sums),
// F32 (fp32 products and sums) or Q8_0 (the input quantized per 32 values,
// exact int32 block sums rescaled in fp32). Without a file the storage
// follows the converters' rules for a weight type (tsk_mmdit_config::
// weight_type). A model whose matrices are all BF16 (the BF16 GGUF; its
// t_embed MLP F32) runs the fused path: glue that the reference emits as
// separate nodes is fused -- LN + modulate + the previous gate * residual
// update (one kernel), qkv split + RMSNorm + RoPE + the F16 cast of K / V +
// the concatenation (the QKV GEMM's epilogue), im2col inside the convolution
// GEMMs, SiLU * gate in the convMLP's epilogue. Other models (Q8_0 with F32
// convolutions, all-F32) keep f32 activations between nodes and convert them
// at each product.
//
// The conditioning that does not depend on t (clip, sync and text input
// projections, the clip_cond / text_cond / global_cond MLP, the clip RoPE
// table) is computed once per sample; each sampler step then runs the
// t-dependent rest and the CFG / Euler update on the device.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/tsk/tsk.h"
#include "host_convert.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

using namespace tsk;

namespace {

enum Kind { K_LIN = 0, K_CONV = 1, K_VEC = 2 };

struct MW {
    std::string name;
    int64_t ne[3];          // ggml ne: linear [in, out]; conv [KW, IC, OC]; vector [n] / [a, b]
    int kind;
    int type;               // storage: TSK_TYPE_F32, TSK_TYPE_BF16 or TSK_TYPE_Q8_0 (vectors F32)
    bool qkv_perm;          // rows (or entries) of a qkv projection: (h d j) -> [q | k | v]
    size_t offset;          // F32 / BF16 values, or the Q8_0 int8 plane [M][K]
    size_t offset_d;        // Q8_0: the fp16 block-scale plane [M][K / 32]
    size_t offset_s;        // split F32 matrix: bf16 planes, rows [hi | lo | hi] per K (per kw for a conv)
    bool split;             // F32 matrix also held as split planes (products as three bf16 ones)
    float amax;             // max |value| of a vector as last set
};

// a linear layer [M][K] in one of the three storage types
struct Lin {
    int type;
    const uint16_t *w;      // BF16
    const float *wf;        // F32
    const int8_t *qw;       // Q8_0 planes
    const uint16_t *dw;
    const uint16_t *ws;     // F32 held split: bf16 rows [M][3 K], [hi | lo | hi]
    const float *b;
    int K, M;
};
// a convolution, kw-major rows [OC][KW * IC] in BF16 or F32
struct Conv {
    int type;
    const uint16_t *w;
    const float *wf;
    const uint16_t *ws;     // F32 held split: bf16 rows [OC][KW * 3 IC], [hi | lo | hi] per kw
    const float *b;
    int KW, IC, OC;
};

struct Block {
    bool pre_only, conv;     // conv: latent / clip streams (k3 linear1 and convMLP)
    int nmod;
    Lin ada, qkv, l1, w1, w3, w2;   // l1 / w1 / w3 / w2 as linear layers (text) ...
    Conv l1c, w1c, w3c, w2c;        // ... or k3 convolutions (latent / clip)
    const float *qn, *kn;
    int qn_idx, kn_idx;
    int64_t mod_col;         // first column of this block's adaLN outputs in its set
};

size_t type_bytes(int type, int64_t n, int plane) {
    if (type == TSK_TYPE_F32) return plane ? 0 : 4 * (size_t) n;
    if (type == TSK_TYPE_BF16) return plane ? 0 : 2 * (size_t) n;
    return plane ? 2 * (size_t) (n / 32) : (size_t) n;     // Q8_0: int8 values, fp16 scales
}

}  // namespace

struct tsk_mmdit {
    tsk_mmdit_config cfg;
    std::vector<MW> w;
    std::unordered_map<std::string, int> idx;
    char *blob = nullptr;
    bool fast = true;                     // every matrix BF16 (t_embed F32): the fused path
    std::vector<Block> jl, jc, jt, fb;   // joint latent / clip / text, fused
    std::vector<float> h_pos_emb, h_empty_str, h_empty_t5;   // host copies for the forward / sampler
    // residual streams (capacity max_batch x max_*); clip0 / txt0 hold the
    // clip and text input projections (t-independent), copied into the
    // streams at the start of every step
    float *lat = nullptr, *clip = nullptr, *txt = nullptr, *sync = nullptr, *ext = nullptr;
    float *clip0 = nullptr, *txt0 = nullptr;
    uint16_t *silu_ext = nullptr, *silu_gc = nullptr;
    float *vec = nullptr;                 // [8][B][H]: te0, te, text_fc, clip_mean, clip_fc, gsum, gcmlp, global_c
    uint16_t *vec16 = nullptr;            // [4][B][max(H, clip_dim)] bf16 vectors
    // adaLN outputs of every block in one pass per forward: the per-token set
    // (latent blocks, then the final layer) [B][T][Ml] and the per-item set
    // (clip blocks, then text blocks) [B][Mg]; Block::mod_col is a block's
    // first column
    float *mods_lat = nullptr, *mods_gc = nullptr;
    Lin ada_lat{}, ada_gc{};              // the blocks' adaLN weights / biases back to back in the blob
    int64_t fin_mod_col = 0;
    uint16_t *xn = nullptr, *hid = nullptr, *o = nullptr, *q = nullptr, *k = nullptr, *vt = nullptr;
    float *part = nullptr, *tmp32 = nullptr, *rope_l = nullptr, *rope_c = nullptr;
    uint16_t *in16 = nullptr;             // bf16 copies of the staged inputs
    float *in32 = nullptr;                // f32 staging of the inputs
    uint16_t *act16 = nullptr;            // bf16(silu(.)) rows of the input projections
    float *freq = nullptr, *temb = nullptr;   // t-embedding frequencies [H / 2] and embeddings [B][H]
    // the f32-activation path: LN outputs, attention output, qkv rows, the
    // SwiGLU hidden state and its halves, and the conversion scratch of the
    // BF16 / Q8_0 products
    float *xn32 = nullptr, *o32 = nullptr, *qkv32 = nullptr, *hid32 = nullptr, *h1 = nullptr, *h3 = nullptr;
    uint16_t *cvt16 = nullptr;
    int8_t *qx = nullptr;
    float *dx = nullptr;
    size_t cvt_cap = 0, q_cap = 0;        // elements of cvt16 / qx
    // sampler state: x token-major [T][L], the step-0 velocity, the flows of one step [2][T][L]
    float *xs = nullptr, *f0 = nullptr, *flow2 = nullptr;
    size_t in_cap = 0;                    // elements of in16 / in32
    int ldv = 0, Nmax = 0, Rmax = 0;
    // stage outputs of the last forward by the reference's debug names
    // (src/mmdit.cpp:333-336), kept while `debug` is set
    bool debug = false;
    std::map<std::string, std::vector<float>> stages;
};

namespace {

int hipcheck(hipError_t e, const char *what) { return e == hipSuccess ? TSK_OK : hip_fail(e, what); }

// debug mode: copy n floats of a device stage tensor to the host under `name`
int grab(tsk_mmdit *m, const char *name, const float *dev, size_t n, hipStream_t st) {
    if (!m->debug) return TSK_OK;
    std::vector<float> v(n);
    hipError_t e = hipStreamSynchronize(st);
    if (e == hipSuccess) e = hipMemcpy(v.data(), dev, sizeof(float) * n, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "debug stage copy");
    m->stages[name].swap(v);
    return TSK_OK;
}

void addw(tsk_mmdit *m, const std::string &name, int64_t a, int64_t b, int64_t c, int kind, bool perm = false) {
    MW x;
    x.name = name;
    x.ne[0] = a; x.ne[1] = b; x.ne[2] = c;
    x.kind = kind;
    x.type = TSK_TYPE_F32;
    x.qkv_perm = perm;
    x.offset = x.offset_d = x.offset_s = 0;
    x.split = false;
    x.amax = 0.0f;
    m->idx[name] = (int) m->w.size();
    m->w.push_back(x);
}

void add_lin(tsk_mmdit *m, const std::string &p, int in, int out, bool bias, bool perm = false) {
    addw(m, p + ".weight", in, out, 1, K_LIN, perm);
    if (bias) addw(m, p + ".bias", out, 1, 1, K_VEC, perm);
}

void add_conv(tsk_mmdit *m, const std::string &p, int kw, int in, int out, bool bias) {
    addw(m, p + ".weight", kw, in, out, K_CONV);
    if (bias) addw(m, p + ".bias", out, 1, 1, K_VEC);
}

// MMDitSingleBlock (docs/ARCHITECTURE.md §6.1): adaLN, qkv, q/k norms, and
// unless pre_only linear1 + ffn (k3 convolutions, or linear layers for text)
void add_block(tsk_mmdit *m, const std::string &p, bool pre_only, bool conv) {
    const int H = m->cfg.hidden, F = m->cfg.mlp_hidden;
    add_lin(m, p + ".adaLN_modulation.1", H, (pre_only ? 2 : 6) * H, true);
    add_lin(m, p + ".attn.qkv", H, 3 * H, true, true);
    addw(m, p + ".attn.q_norm.weight", m->cfg.head_dim, 1, 1, K_VEC);
    addw(m, p + ".attn.k_norm.weight", m->cfg.head_dim, 1, 1, K_VEC);
    if (pre_only) return;
    if (conv) {
        add_conv(m, p + ".linear1", 3, H, H, true);
        add_conv(m, p + ".ffn.w1", 3, H, F, false);
        add_conv(m, p + ".ffn.w3", 3, H, F, false);
        add_conv(m, p + ".ffn.w2", 3, F, H, false);
    } else {
        add_lin(m, p + ".linear1", H, H, true);
        add_lin(m, p + ".ffn.w1", H, F, false);
        add_lin(m, p + ".ffn.w3", H, F, false);
        add_lin(m, p + ".ffn.w2", F, H, false);
    }
}

// The storage type of a weight under a model-wide weight type, as the
// converters write the files: the BF16 GGUF casts linears and convolutions
// to BF16 but keeps "_emb" names (the t_embed MLP) F32; the Q8_0 GGUF
// quantizes the 2-D linears with ne0 % 32 == 0 whose names hold none of
// "_emb", "norm", "empty" and keeps the 3-D convolution kernels F32
// (convert/quantize_gguf.py:9-15); the F32 GGUF keeps every tensor F32
// (convert/convert_thinksound.py:55-57). Vectors are F32 in every file.
int rule_type(int weight_type, const MW &x) {
    if (x.kind == K_VEC || weight_type == TSK_TYPE_F32) return TSK_TYPE_F32;
    const bool emb = x.name.find("_emb") != std::string::npos;
    if (weight_type == TSK_TYPE_BF16) return emb ? TSK_TYPE_F32 : TSK_TYPE_BF16;
    if (x.kind == K_CONV || emb || x.name.find("norm") != std::string::npos ||
        x.name.find("empty") != std::string::npos || x.ne[0] % 32)
        return TSK_TYPE_F32;
    return TSK_TYPE_Q8_0;
}

const MW &wi(const tsk_mmdit *m, const std::string &n) { return m->w[m->idx.at(n)]; }
template <class T> T *wp(const tsk_mmdit *m, const std::string &n) { return (T *) (m->blob + wi(m, n).offset); }

Lin lin_of(const tsk_mmdit *m, const std::string &p, bool bias) {
    const MW &x = wi(m, p + ".weight");
    Lin L;
    memset(&L, 0, sizeof(L));
    L.type = x.type;
    L.K = (int) x.ne[0];
    L.M = (int) x.ne[1];
    char *base = m->blob + x.offset;
    if (x.type == TSK_TYPE_F32) L.wf = (const float *) base;
    else if (x.type == TSK_TYPE_BF16) L.w = (const uint16_t *) base;
    else { L.qw = (const int8_t *) base; L.dw = (const uint16_t *) (m->blob + x.offset_d); }
    if (x.split) L.ws = (const uint16_t *) (m->blob + x.offset_s);
    L.b = bias ? wp<float>(m, p + ".bias") : nullptr;
    return L;
}

Conv conv_of(const tsk_mmdit *m, const std::string &p, bool bias) {
    const MW &x = wi(m, p + ".weight");
    Conv C;
    memset(&C, 0, sizeof(C));
    C.type = x.type;
    if (x.type == TSK_TYPE_F32) C.wf = wp<float>(m, p + ".weight");
    else C.w = wp<uint16_t>(m, p + ".weight");
    if (x.split) C.ws = (const uint16_t *) (m->blob + x.offset_s);
    C.b = bias ? wp<float>(m, p + ".bias") : nullptr;
    C.KW = (int) x.ne[0];
    C.IC = (int) x.ne[1];
    C.OC = (int) x.ne[2];
    return C;
}

Block block_of(const tsk_mmdit *m, const std::string &p, bool pre_only, bool conv) {
    Block b;
    memset(&b, 0, sizeof(b));
    b.pre_only = pre_only;
    b.conv = conv;
    b.nmod = pre_only ? 2 : 6;
    b.ada = lin_of(m, p + ".adaLN_modulation.1", true);
    b.qkv = lin_of(m, p + ".attn.qkv", true);
    b.qn = wp<float>(m, p + ".attn.q_norm.weight");
    b.kn = wp<float>(m, p + ".attn.k_norm.weight");
    b.qn_idx = m->idx.at(p + ".attn.q_norm.weight");
    b.kn_idx = m->idx.at(p + ".attn.k_norm.weight");
    if (!pre_only) {
        if (conv) {
            b.l1c = conv_of(m, p + ".linear1", true);
            b.w1c = conv_of(m, p + ".ffn.w1", false);
            b.w3c = conv_of(m, p + ".ffn.w3", false);
            b.w2c = conv_of(m, p + ".ffn.w2", false);
        } else {
            b.l1 = lin_of(m, p + ".linear1", true);
            b.w1 = lin_of(m, p + ".ffn.w1", false);
            b.w3 = lin_of(m, p + ".ffn.w3", false);
            b.w2 = lin_of(m, p + ".ffn.w2", false);
        }
    }
    return b;
}

int validate_cfg(const tsk_mmdit_config *c) {
    if (!c) return fail(TSK_ERR_INVALID_ARG, "cfg is NULL");
    if (c->head_dim != 64 || c->hidden != c->n_head * 64) return fail(TSK_ERR_UNSUPPORTED, "head_dim must be 64, hidden = 64 n_head");
    if (c->hidden % 64 || c->mlp_hidden % 64 || c->latent_dim % 32 || c->latent_dim < 32 || c->clip_dim % 64 ||
        c->sync_dim % 64 || c->t5_dim % 64 || c->t5_dim < c->clip_dim)
        return fail(TSK_ERR_SHAPE, "hidden, mlp_hidden, clip / sync / t5 dims must be multiples of 64, latent_dim of 32");
    if (c->depth - c->fused_depth < 1 || c->fused_depth < 0) return fail(TSK_ERR_SHAPE, "depth / fused_depth");
    if (c->max_batch < 1 || c->max_batch > 32 || c->max_latent < 1 || c->max_clip < 1 || c->max_sync < 8 ||
        c->text_seq < 1)
        return fail(TSK_ERR_SHAPE, "capacity");
    if (!(c->rope_theta > 0) || !(c->t_max_period > 0)) return fail(TSK_ERR_INVALID_ARG, "rope_theta / t_max_period");
    if (c->weight_type != TSK_TYPE_BF16 && c->weight_type != TSK_TYPE_Q8_0 && c->weight_type != TSK_TYPE_F32)
        return fail(TSK_ERR_TYPE, "weight_type %d: TSK_TYPE_BF16, TSK_TYPE_Q8_0 or TSK_TYPE_F32", c->weight_type);
    return TSK_OK;
}

// ---- GEMMs of the fused path (bf16 activation rows, launch_gemm_coop)

// y[n][m] = x[n] . W[m] + b with an F32 weight: f32 activations, fp32 products
int lin_f32(const Lin &L, const float *x, int N, float *y, hipStream_t s) {
    GemmProblem q;
    memset(&q, 0, sizeof(q));
    q.x = x; q.ld_x = L.K;
    q.wf = L.wf; q.ld_w = L.K;
    q.bias = L.b;
    q.y = y; q.ld_y = L.M;
    q.M = L.M; q.N = N; q.K = L.K; q.splits = 1;
    return hipcheck(launch_gemm_f32(q, 0, s), "mmdit f32 linear");
}

// y[n][m] = x[n] . W[m] (+ b): x bf16 rows (ld_x), y f32 or bf16 rows (ld_y)
int lin(const Lin &L, const uint16_t *x, int64_t ld_x, int N, void *y, int64_t ld_y, bool y_bf16, hipStream_t s,
        const float *bias_override = nullptr, bool no_bias = false) {
    GemmGroup g;
    memset(&g, 0, sizeof(g));
    g.nprob = 1;
    GemmProblem &q = g.p[0];
    q.x = x; q.ld_x = ld_x;
    q.w = L.w; q.ld_w = L.K;
    q.bias = no_bias ? nullptr : bias_override ? bias_override : L.b;
    q.y = y; q.ld_y = ld_y;
    q.M = L.M; q.N = N; q.K = L.K; q.splits = 1;
    return hipcheck(launch_gemm_coop(g, y_bf16 ? EPI_STORE_BF16 : EPI_STORE_F32, s), "mmdit linear");
}

// conv_cl (stride 1, padding pad): x bf16 rows [B][IW][IC] with row stride
// ld_x and batch stride xb (elements), y rows [B * IW][OC] (ld_y)
GemmProblem conv_problem(const Conv &C, const uint16_t *x, int64_t ld_x, int64_t xb, int IW, int B, int pad, void *y,
                         int64_t ld_y, bool no_bias, int splits) {
    GemmProblem q;
    memset(&q, 0, sizeof(q));
    q.x = x; q.ld_x = ld_x; q.x_group_stride = xb;
    q.w = C.w; q.ld_w = (int64_t) C.KW * C.IC;
    q.bias = no_bias ? nullptr : C.b;
    q.y = y; q.ld_y = ld_y;
    const int OW = IW + 2 * pad - (C.KW - 1);
    q.M = C.OC; q.N = B * OW; q.K = C.KW * C.IC; q.splits = splits;
    q.conv_ic = C.IC; q.conv_iw = IW; q.conv_ow = OW; q.conv_s = 1; q.conv_p = pad; q.conv_d = 1;
    return q;
}

int conv(const Conv &C, const uint16_t *x, int64_t ld_x, int64_t xb, int IW, int B, int pad, void *y, int64_t ld_y,
         bool y_bf16, hipStream_t s, bool no_bias = false, int splits = 1) {
    GemmGroup g;
    memset(&g, 0, sizeof(g));
    g.nprob = 1;
    g.p[0] = conv_problem(C, x, ld_x, xb, IW, B, pad, y, ld_y, no_bias, splits);
    const int epi = splits > 1 ? EPI_PARTIAL : y_bf16 ? EPI_STORE_BF16 : EPI_STORE_F32;
    return hipcheck(launch_gemm_coop(g, epi, s), "mmdit conv");
}

// K slices of a residual-branch convolution (linear1, convMLP w2) whose
// partial sums the next LayerNorm adds up: with few output tiles (1024
// outputs x 388 rows at 9 s is 112 tiles of 64 x 64) each workgroup would
// stream all of K = 3072 / 8448 alone; the slices fill the 256 CUs (up to
// three workgroups each). The count follows from the rows per batch item
// times the model's batch capacity, never from the call's batch: a batch row
// is then summed in the same order whatever the batch it runs in. At most
// TSK_GRAPH_KSPLIT slices (4) below TSK_GRAPH_KSWG workgroups (1536: the
// 30 s step 6.04 -> 5.90 ms against 768; 8 slices or 3072 no better).
// K slices of the f32 path's F32 products (gemm_f32's 128 x 64 tiles): the
// Q8_0 GGUF keeps the convolution kernels F32, and linear1 / convMLP w2 with
// 1024 outputs over a few hundred rows are 56-168 tiles with K = 3072 / 8448;
// slices of at least 256 k until about 2000 workgroups (swept: 8 slices were
// the fastest for every graph shape but the 30 s latent w1 / w3, best at 4),
// by the rows per batch item times the batch capacity (never by the call's
// batch)
constexpr int F32_KSPLIT_MAX = 8;
constexpr int PART_SLICES = 8;      // partial-sum slices per stream row in m->part (either path)
int f32_splits(const tsk_mmdit *m, int M, int K, int S) {
    const int N = S * m->cfg.max_batch;
    const int64_t tiles = (int64_t) ((M + 127) / 128) * ((N + 63) / 64);
    const int nk = (K + 31) / 32;
    int sp = 1;
    const int most = std::min(F32_KSPLIT_MAX, std::max(1, tuning().f32_ksplit));
    while (sp * 2 <= most && tiles * sp * 2 <= 2048 && nk / (2 * sp) >= 8) sp *= 2;
    return sp;
}

int conv_splits(const tsk_mmdit *m, const Conv &C, int S) {
    const int N = S * m->cfg.max_batch;
    const int64_t tiles = (int64_t) ((C.OC + 63) / 64) * ((N + 63) / 64);
    const int kt = C.KW * C.IC / 32;
    int sp = 1;
    const int most = std::min(PART_SLICES, std::max(1, tuning().graph_ksplit));
    while (sp * 2 <= most && tiles * sp * 2 <= tuning().graph_ks_wg && kt % (2 * sp) == 0 && (kt / (2 * sp)) % 2 == 0)
        sp *= 2;
    return sp;
}

int conv_plain(tsk_mmdit *m, const Conv &C, const uint16_t *x, int64_t ld_x, int64_t xb, int IW, int B, int pad,
               float *y, int64_t ld_y, bool bias, hipStream_t s);

// convmlp / mlp (src/mmdit.cpp:39-52): y = w2(silu(w1 x) * w3 x), the hidden
// state bf16 in m->hid (the conversion w2's mul_mat applies to it); w2 into
// residual slices (splits > 1) or plain rows
int conv_mlp(tsk_mmdit *m, const Conv &w1, const Conv &w3, const Conv &w2, const uint16_t *x, int64_t ld_x, int64_t xb,
             int IW, int B, float *y, int64_t ld_y, hipStream_t s, int splits = 1) {
    GemmGroup g;
    memset(&g, 0, sizeof(g));
    g.nprob = 1;
    GemmProblem &q = g.p[0];
    q.x = x; q.ld_x = ld_x; q.x_group_stride = xb;
    q.w = w1.w; q.w3 = w3.w; q.ld_w = (int64_t) w1.KW * w1.IC;
    q.y = m->hid; q.ld_y = w1.OC;
    q.M = w1.OC; q.N = B * IW; q.K = w1.KW * w1.IC; q.splits = 1;
    q.conv_ic = w1.IC; q.conv_iw = IW; q.conv_ow = IW; q.conv_s = 1; q.conv_p = 1; q.conv_d = 1;
    int rc = hipcheck(launch_gemm_coop(g, EPI_SWIGLU_BF16, s), "mmdit convmlp w1/w3");
    if (rc) return rc;
    if (splits == 1) return conv_plain(m, w2, m->hid, w1.OC, (int64_t) IW * w1.OC, IW, B, 1, y, ld_y, false, s);
    return conv(w2, m->hid, w1.OC, (int64_t) IW * w1.OC, IW, B, 1, y, ld_y, false, s, true, splits);
}

int lin_mlp(tsk_mmdit *m, const Lin &w1, const Lin &w3, const Lin &w2, const uint16_t *x, int64_t ld_x, int N, float *y,
            int64_t ld_y, hipStream_t s) {
    GemmGroup g;
    memset(&g, 0, sizeof(g));
    g.nprob = 1;
    GemmProblem &q = g.p[0];
    q.x = x; q.ld_x = ld_x;
    q.w = w1.w; q.w3 = w3.w; q.ld_w = w1.K;
    q.y = m->hid; q.ld_y = w1.M;
    q.M = w1.M; q.N = N; q.K = w1.K; q.splits = 1;
    int rc = hipcheck(launch_gemm_coop(g, EPI_SWIGLU_BF16, s), "mmdit mlp w1/w3");
    if (rc) return rc;
    return lin(w2, m->hid, w1.M, N, y, ld_y, false, s, nullptr, true);
}

// ---- products of the f32-activation path: f32 rows in, f32 rows out, the
// input converted to the weight's vec_dot type as ggml_mul_mat does

// N rows of f32 activations: row n at x + (n / grp) * gstride + (n % grp) * ld
// (grp = 0: x + n * ld)
struct Rows {
    const float *x;
    int64_t ld;
    int grp;
    int64_t gstride;
};

// the rows as contiguous bf16 [N][K] in m->cvt16
int rows_bf16(tsk_mmdit *m, const Rows &src, int N, int K, hipStream_t s) {
    if ((size_t) N * K > m->cvt_cap) return fail(TSK_ERR_SHAPE, "bf16 conversion of %d x %d exceeds the scratch", N, K);
    const int rpb = src.grp ? src.grp : N;
    return hipcheck(launch_cast_rows_bf16(src.x, src.ld, src.grp ? src.gstride : 0, rpb, N, K, m->cvt16, s),
                    "mmdit bf16 rows");
}

// F32 products as three bf16 ones (TSK_F32_SPLIT, for a model created with
// it): the weight's planes [hi | lo | hi] against the rows' [hi | hi | lo]
// sum x_hi w_hi + x_hi w_lo + x_lo w_hi over 3 K, which leaves out x_lo w_lo
// and the roundings of the lo parts, about 2^-17 of |x w| per term (fp32
// MFMA products: 157 TFLOP/s at most; three bf16 ones: 2.5 PFLOP/s / 3)
bool split_on(const uint16_t *ws) { return ws && tuning().f32_split; }
Lin split_lin(const Lin &L) {
    Lin S = L;
    S.type = TSK_TYPE_BF16; S.w = L.ws; S.K = 3 * L.K;
    return S;
}
Conv split_conv(const Conv &C) {
    Conv S = C;
    S.type = TSK_TYPE_BF16; S.w = C.ws; S.IC = 3 * C.IC;
    return S;
}
// the rows as the split operand [N][3 K] in m->cvt16
int rows_split3(tsk_mmdit *m, const Rows &src, int N, int K, hipStream_t s) {
    if ((size_t) N * 3 * K > m->cvt_cap) return fail(TSK_ERR_SHAPE, "split rows of %d x %d exceed the scratch", N, K);
    const int rpb = src.grp ? src.grp : N;
    return hipcheck(launch_cast_rows_split3(src.x, src.ld, src.grp ? src.gstride : 0, rpb, N, K, m->cvt16, s),
                    "mmdit split rows");
}
// K slices of a split product (K three times the F32 one, 9216-25344 for
// the graph's convolutions): the most, up to `most`, that keep the 128 x 128
// tiles times slices within TSK_SPLIT_WG (512; swept 256-1536 on the Q8_0
// graph: 384-512 best, 9 s 7.26 against 7.57-7.80 ms per forward, 30 s
// 12.24 against 13.05-13.12); every slice an even number of 32-k tiles.
// Counted from the rows per batch item times the batch capacity, so that a
// batch row is summed in the same order whatever the call's batch.
int split_slices(const tsk_mmdit *m, int M, int K, int S, int most = PART_SLICES) {
    const int64_t t = (int64_t) ((M + 127) / 128) * ((S * m->cfg.max_batch + 127) / 128);
    const int kt = K / 32;
    int sp = 1;
    for (int c = 2; c <= most; ++c)
        if (kt % c == 0 && (kt / c) % 2 == 0 && t * c <= tuning().split_wg) sp = c;
    return sp;
}
constexpr int SPLIT_SUM_MAX = 16;   // slices of a split convolution summed into a plain output
// A BF16 convolution into plain f32 rows (y = conv(x) + b): over few tiles
// with a long K (the input projections' convMLP w2, K = 8448 over 112
// workgroups at 9 s; the final k7 convolution, 64 outputs, 7 workgroups) as
// K-split slices in m->part, summed with the bias by sum_slices_kernel. Only
// between blocks: no residual partial sums are pending in m->part then.
int conv_plain(tsk_mmdit *m, const Conv &C, const uint16_t *x, int64_t ld_x, int64_t xb, int IW, int B, int pad,
               float *y, int64_t ld_y, bool bias, hipStream_t s) {
    const int OW = IW + 2 * pad - (C.KW - 1), N = B * OW;
    const int64_t rows3 = (int64_t) m->cfg.max_batch * (m->cfg.max_latent + m->cfg.max_clip + 2 * m->cfg.text_seq);
    const size_t cap = (size_t) PART_SLICES * rows3 * m->cfg.hidden;   // floats of m->part
    const int most = (int) std::min<size_t>(SPLIT_SUM_MAX, cap / ((size_t) m->cfg.max_batch * OW * C.OC));
    const int sp = C.OC % 4 == 0 && ld_y % 4 == 0 && ((uintptr_t) y & 15) == 0
                       ? split_slices(m, C.OC, C.KW * C.IC, OW, most) : 1;
    if (sp == 1) return conv(C, x, ld_x, xb, IW, B, pad, y, ld_y, false, s, !bias);
    int rc = conv(C, x, ld_x, xb, IW, B, pad, m->part, C.OC, false, s, true, sp);
    if (rc) return rc;
    return hipcheck(launch_sum_slices(m->part, sp, (int64_t) N * C.OC, bias ? C.b : nullptr, N, C.OC, y, ld_y, s),
                    "mmdit conv slices");
}

// K slices of a residual-branch convolution on the f32 path (summed by the
// next LayerNorm): F32 kernels as fp32 products by f32_splits, as split
// products by split_slices; BF16 kernels unsplit
int res_splits(const tsk_mmdit *m, const Conv &C, int S) {
    if (C.type != TSK_TYPE_F32) return 1;
    return split_on(C.ws) ? split_slices(m, C.OC, 3 * C.KW * C.IC, S) : f32_splits(m, C.OC, C.KW * C.IC, S);
}

// y[n][m] = x[n] . W[m] (+ b), any storage type
// qs (Q8_0 weights only): the rows go to the attention operands through the
// GEMM's QKV epilogue instead of y (the caller's scatter is then skipped)
int g_lin(tsk_mmdit *m, const Lin &L, const Rows &src, int N, float *y, int64_t ld_y, bool bias, hipStream_t s,
          const QkvScatter *qs = nullptr) {
    const float *b = bias ? L.b : nullptr;
    if (L.type == TSK_TYPE_F32 && split_on(L.ws)) {
        int rc = rows_split3(m, src, N, L.K, s);
        if (rc) return rc;
        return lin(split_lin(L), m->cvt16, 3 * L.K, N, y, ld_y, false, s, nullptr, !bias);
    }
    if (L.type == TSK_TYPE_F32) {
        GemmProblem q;
        memset(&q, 0, sizeof(q));
        q.x = src.x; q.ld_x = src.ld; q.x_group_rows = src.grp; q.x_group_stride = src.gstride;
        q.wf = L.wf; q.ld_w = L.K;
        q.bias = b;
        q.y = y; q.ld_y = ld_y;
        q.M = L.M; q.N = N; q.K = L.K; q.splits = 1;
        return hipcheck(launch_gemm_f32(q, 0, s), "mmdit f32 linear");
    }
    if (L.type == TSK_TYPE_BF16) {
        int rc = rows_bf16(m, src, N, L.K, s);
        if (rc) return rc;
        return lin(L, m->cvt16, L.K, N, y, ld_y, false, s, nullptr, !bias);
    }
    // Q8_0: the rows quantized per 32 (ggml-cpu's x86 rounding), int8 MFMA.
    // The quantizer's group stride counts rows of ld_x, not elements.
    if ((size_t) N * L.K > m->q_cap) return fail(TSK_ERR_SHAPE, "Q8_0 conversion of %d x %d exceeds the scratch", N, L.K);
    if (src.grp && src.gstride % src.ld)
        return fail(TSK_ERR_STRIDE, "Q8_0 rows: group stride %lld is not a multiple of the row stride %lld",
                    (long long) src.gstride, (long long) src.ld);
    hipError_t e = launch_quantize_rows_q8(src.x, 1, src.ld, N, L.K, m->qx, m->dx, s, src.grp,
                                           src.grp ? src.gstride / src.ld : 0);
    if (e != hipSuccess) return hip_fail(e, "mmdit q8_0 quantize");
    GemmParams p;
    memset(&p, 0, sizeof(p));
    p.qw = L.qw; p.dw = L.dw;
    p.qx = m->qx; p.dx = m->dx;
    p.M = L.M; p.N = N; p.K = L.K;
    p.bias = b;
    p.y = y; p.ld_y = ld_y;
    p.epi = EPI_STORE;
    if (qs) {
        p.epi = EPI_QKV_ATTN;
        p.qs = *qs;
    }
    p.rows_per_gate = 1;
    p.splits = 1;
    return hipcheck(launch_gemm_q8(p, s), "mmdit q8_0 linear");
}

// conv_cl (stride 1, padding pad) of f32 rows [B][IW][IC] (row stride ld_x,
// batch stride xb) -> f32 rows [B * OW][OC] (ld_y), or with splits > 1 (no
// bias) K-split partial sums in slices [splits][B * OW][ld_y]
int g_conv(tsk_mmdit *m, const Conv &C, const float *x, int64_t ld_x, int64_t xb, int IW, int B, int pad, float *y,
           int64_t ld_y, bool bias, hipStream_t s, int splits = 1) {
    if (splits > 1 && bias) return fail(TSK_ERR_INVALID_ARG, "K-split slices carry no bias");
    if (C.type == TSK_TYPE_F32 && split_on(C.ws)) {
        int rc = rows_split3(m, Rows{x, ld_x, IW, xb}, B * IW, C.IC, s);
        if (rc) return rc;
        const Conv S = split_conv(C);
        // a plain output over few tiles (the input projections' and the final
        // layer's convolutions, up to K = 25344): K-split slices into m->h3
        // (free outside the SwiGLU halves), summed with the bias
        const int OW = IW + 2 * pad - (C.KW - 1), N = B * OW;
        const size_t cap = (size_t) F32_KSPLIT_MAX * m->Rmax * m->cfg.mlp_hidden;   // floats of m->h3
        const int most = (int) std::min<size_t>(SPLIT_SUM_MAX, cap / ((size_t) m->cfg.max_batch * OW * C.OC));
        const int sp = splits == 1 && C.OC % 4 == 0 && ld_y % 4 == 0 && ((uintptr_t) y & 15) == 0
                           ? split_slices(m, C.OC, S.KW * S.IC, OW, most) : 1;
        if (sp > 1) {
            if ((rc = conv(S, m->cvt16, S.IC, (int64_t) IW * S.IC, IW, B, pad, m->h3, C.OC, false, s, true, sp)))
                return rc;
            return hipcheck(launch_sum_slices(m->h3, sp, (int64_t) N * C.OC, bias ? C.b : nullptr, N, C.OC, y, ld_y, s),
                            "mmdit split slices");
        }
        return conv(S, m->cvt16, S.IC, (int64_t) IW * S.IC, IW, B, pad, y, ld_y, false, s, !bias, splits);
    }
    if (C.type == TSK_TYPE_F32) {
        GemmProblem q;
        memset(&q, 0, sizeof(q));
        q.x = x; q.ld_x = ld_x; q.x_group_stride = xb;
        q.wf = C.wf; q.ld_w = (int64_t) C.KW * C.IC;
        q.bias = bias ? C.b : nullptr;
        q.y = y; q.ld_y = ld_y;
        const int OW = IW + 2 * pad - (C.KW - 1);
        q.M = C.OC; q.N = B * OW; q.K = C.KW * C.IC; q.splits = splits;
        q.conv_ic = C.IC; q.conv_iw = IW; q.conv_ow = OW; q.conv_s = 1; q.conv_p = pad; q.conv_d = 1;
        return hipcheck(launch_gemm_f32(q, 0, s), "mmdit f32 conv");
    }
    const Rows src{x, ld_x, IW, xb};
    int rc = rows_bf16(m, src, B * IW, C.IC, s);
    if (rc) return rc;
    return conv(C, m->cvt16, C.IC, (int64_t) IW * C.IC, IW, B, pad, y, ld_y, false, s, !bias, splits);
}

// convmlp / mlp (src/mmdit.cpp:39-52) on f32 rows: y = w2(silu(w1 x) * w3 x)
// (no biases), the hidden state f32 in m->hid32. Convolutions (conv: rows
// [B][S][IC], batch stride xb) or linear layers (x rows of B * S). F32
// convolution halves w1 / w3 run as K-split slices (summed by the SiLU * gate
// kernel); w2 writes y2_splits slices of partial sums (conv, 1: plain y).
int g_swiglu(tsk_mmdit *m, bool is_conv, const Conv &c1, const Conv &c3, const Conv &c2, const Lin &l1, const Lin &l3,
             const Lin &l2, const float *x, int64_t ld_x, int64_t xb, int S, int B, float *y, int64_t ld_y,
             hipStream_t s, int y2_splits = 1) {
    const int N = B * S;
    const int F = is_conv ? c1.OC : l1.M;
    const int t1 = is_conv ? c1.type : l1.type, t3 = is_conv ? c3.type : l3.type;
    const bool split = t1 == TSK_TYPE_F32 && t3 == TSK_TYPE_F32 && split_on(is_conv ? c1.ws : l1.ws) &&
                       split_on(is_conv ? c3.ws : l3.ws);
    // split convolution halves over few rows (the 9 s shapes: 176 tiles of
    // 128 x 128 where the fused GEMM would take 64 x 64 ones streaming all of
    // K = 9216): each half as K-split slices of 128-row tiles, summed by the
    // SiLU * gate kernel
    const bool split_sliced = split && is_conv && (int64_t) ((F + 63) / 64) * ((N + 127) / 128) < 400;
    int rc;
    if (split_sliced) {
        const int IC = 3 * c1.IC;
        const int sp = split_slices(m, F, c1.KW * IC, S);
        if ((rc = rows_split3(m, Rows{x, ld_x, S, xb}, N, c1.IC, s))) return rc;
        if ((rc = conv(split_conv(c1), m->cvt16, IC, (int64_t) S * IC, S, B, 1, m->h1, F, false, s, true, sp)) ||
            (rc = conv(split_conv(c3), m->cvt16, IC, (int64_t) S * IC, S, B, 1, m->h3, F, false, s, true, sp)) ||
            (rc = hipcheck(launch_silu_mul_slices(m->h1, m->h3, sp, (int64_t) N * F, m->hid32, (int64_t) N * F, s),
                           "mmdit silu * gate")))
            return rc;
    } else if ((t1 == TSK_TYPE_BF16 && t3 == TSK_TYPE_BF16) || split) {
        // both halves in one cooperative GEMM with the SwiGLU epilogue, f32
        // out; split F32 halves over their planes and the rows' split operand
        const int f = split ? 3 : 1, IC = f * (is_conv ? c1.IC : l1.K);
        const Rows src = is_conv ? Rows{x, ld_x, S, xb} : Rows{x, ld_x, 0, 0};
        if ((rc = split ? rows_split3(m, src, N, IC / 3, s) : rows_bf16(m, src, N, IC, s))) return rc;
        GemmGroup g;
        memset(&g, 0, sizeof(g));
        g.nprob = 1;
        GemmProblem &q = g.p[0];
        q.x = m->cvt16; q.ld_x = IC;
        q.w = split ? (is_conv ? c1.ws : l1.ws) : is_conv ? c1.w : l1.w;
        q.w3 = split ? (is_conv ? c3.ws : l3.ws) : is_conv ? c3.w : l3.w;
        q.ld_w = is_conv ? (int64_t) c1.KW * IC : IC;
        q.y = m->hid32; q.ld_y = F;
        q.M = F; q.N = N; q.K = (int) q.ld_w; q.splits = 1;
        if (is_conv) {
            q.x_group_stride = (int64_t) S * IC;
            q.conv_ic = IC; q.conv_iw = S; q.conv_ow = S; q.conv_s = 1; q.conv_p = 1; q.conv_d = 1;
        }
        if ((rc = hipcheck(launch_gemm_coop(g, EPI_SWIGLU_F32, s), "mmdit swiglu w1/w3"))) return rc;
    } else {
        int sp = 1;
        if (is_conv) {
            if (t1 == TSK_TYPE_F32 && t3 == TSK_TYPE_F32) sp = f32_splits(m, F, c1.KW * c1.IC, S);
            if ((rc = g_conv(m, c1, x, ld_x, xb, S, B, 1, m->h1, F, false, s, sp)) ||
                (rc = g_conv(m, c3, x, ld_x, xb, S, B, 1, m->h3, F, false, s, sp)))
                return rc;
        } else {
            const Rows src{x, ld_x, 0, 0};
            if ((rc = g_lin(m, l1, src, N, m->h1, F, false, s)) || (rc = g_lin(m, l3, src, N, m->h3, F, false, s)))
                return rc;
        }
        if ((rc = hipcheck(launch_silu_mul_slices(m->h1, m->h3, sp, (int64_t) N * F, m->hid32, (int64_t) N * F, s),
                           "mmdit silu * gate")))
            return rc;
    }
    if (is_conv) return g_conv(m, c2, m->hid32, F, (int64_t) S * F, S, B, 1, y, ld_y, false, s, y2_splits);
    return g_lin(m, l2, Rows{m->hid32, F, 0, 0}, N, y, ld_y, false, s);
}

int g_conv_mlp(tsk_mmdit *m, const std::string &p, const float *x, int64_t ld_x, int64_t xb, int S, int B, float *y,
               int64_t ld_y, hipStream_t s) {
    const Lin none{};
    return g_swiglu(m, true, conv_of(m, p + ".w1", false), conv_of(m, p + ".w3", false), conv_of(m, p + ".w2", false),
                    none, none, none, x, ld_x, xb, S, B, y, ld_y, s);
}

int g_lin_mlp(tsk_mmdit *m, const std::string &p, const float *x, int64_t ld_x, int N, float *y, int64_t ld_y,
              hipStream_t s) {
    const Conv none{};
    return g_swiglu(m, false, none, none, none, lin_of(m, p + ".w1", false), lin_of(m, p + ".w3", false),
                    lin_of(m, p + ".w2", false), x, ld_x, 0, N, 1, y, ld_y, s);
}

// ---- one stream of a block as the fused kernels see it
struct Stream {
    const Block *w;
    float *x;              // f32 residual rows [B][S][H]
    int S, tok_off;
    const float *rope_cs;  // nullptr: no RoPE (text)
    float *mod;            // this block's adaLN outputs: [B * rows_mod] rows of stride ld_mod
    int64_t ld_mod;
    int per_token;         // modulation per token (latent: extended_c) or per batch item
    void *xn;              // LN output rows: bf16 (fused path) or f32
    float *part;           // f32 output of the previous projection (residual update owed)
    const float *pend_bias, *pend_gate;
    int64_t pend_ld;       // row stride of pend_gate (the owing block's adaLN width)
    int pend_split;        // K slices of part ([split][B S][H]) the owed update is summed from
    bool pending;
};

LnStream ln_of(const tsk_mmdit *m, Stream &r, int B, int which) {
    const int H = m->cfg.hidden;
    LnStream l;
    memset(&l, 0, sizeof(l));
    l.x = r.x; l.ld_x = H;
    const int64_t ldm = r.ld_mod;
    if (r.pending) {
        l.part = r.part; l.nsplit = r.pend_split > 1 ? r.pend_split : 1; l.part_stride = (int64_t) B * r.S * H;
        l.bias = r.pend_bias; l.gate = r.pend_gate; l.ld_gate = r.pend_ld;
        r.pending = false;
    }
    l.shift = r.mod + (which ? 3 : 0) * H;
    l.scale = r.mod + (which ? 4 : 1) * H;
    l.ld_mod = ldm;
    l.y = r.xn; l.ld_y = H;
    l.rows = B * r.S;
    l.rows_per_b = r.per_token ? 1 : r.S;
    return l;
}

// LN(which) of up to three streams (two per launch): bf16 rows on the fused
// path, f32 rows otherwise
int run_ln(tsk_mmdit *m, Stream *r, int ns, int B, int which, hipStream_t s) {
    for (int i0 = 0; i0 < ns; i0 += 2) {
        LnGroup g;
        memset(&g, 0, sizeof(g));
        g.H = m->cfg.hidden;
        g.eps = 1e-5f;                                   // layernorm() eps, src/mmdit.cpp:59
        g.y_mode = m->fast ? LN_Y_BF16 : LN_Y_F32;
        g.nstream = ns - i0 >= 2 ? 2 : 1;
        for (int j = 0; j < g.nstream; ++j) g.s[j] = ln_of(m, r[i0 + j], B, which);
        int rc = hipcheck(launch_ln_group(g, s), "mmdit layernorm");
        if (rc) return rc;
    }
    return TSK_OK;
}

constexpr float QK_EPS = 1e-6f;                                      // rmsnorm_w EPS, src/mmdit.cpp:10
constexpr float Q_SCALE = 1.4426950408889634f / 8.0f;                 // 1/sqrt(64) * log2(e): the softmax scale

// tiles of the QKV GEMM: 128 x 64 from 1100 activation rows, 64 x 64 below
// (the DiT's qkv rule)
int qkv_cfg(int rows) { return rows >= 1100 ? 29 : 30; }

// qkv with the split / RMSNorm / RoPE / F16 scatter into the joint attention
// operands in the GEMM epilogue (EPI_QKV); up to two streams per launch
int run_qkv(tsk_mmdit *m, Stream *r, int ns, int B, int Ntot, hipStream_t s) {
    const tsk_mmdit_config &c = m->cfg;
    const int H = c.hidden;
    for (int i0 = 0; i0 < ns; i0 += 2) {
        GemmGroup g;
        memset(&g, 0, sizeof(g));
        g.nprob = std::min(2, ns - i0);
        int rows0 = 0;
        for (int k = 0; k < g.nprob; ++k) {
            const Stream &st = r[i0 + k];
            const Lin &L = st.w->qkv;
            GemmProblem &q = g.p[k];
            q.x = st.xn; q.ld_x = H;
            q.w = L.w; q.ld_w = L.K;
            q.bias = L.b;
            q.M = L.M; q.N = B * st.S; q.K = L.K; q.splits = 1;
            q.qn_w = st.w->qn; q.kn_w = st.w->kn;
            q.q = m->q; q.k = m->k; q.vt = m->vt; q.ldv = m->ldv;
            q.v_rows = tuning().attn_vrows != 0;   // V as rows like k
            q.seq = st.S; q.Ntot = Ntot; q.tok_off = st.tok_off;
            q.rope = st.rope_cs != nullptr;
            q.rope_cs = st.rope_cs;
            q.eps = QK_EPS;
            q.q_scale = Q_SCALE;
            rows0 = std::max(rows0, q.N);
        }
        const int rc = hipcheck(launch_gemm_ks(g, EPI_QKV, qkv_cfg(rows0), s), "mmdit qkv gemm");
        if (rc) return rc;
    }
    return TSK_OK;
}

// the f32 path: qkv rows (bias included) then the split / RMSNorm / RoPE /
// F16 scatter kernel, per stream; with Q8_0 weights the scatter runs as the
// GEMM's epilogue
int run_qkv_f32(tsk_mmdit *m, Stream *r, int ns, int B, int Ntot, hipStream_t s) {
    const tsk_mmdit_config &c = m->cfg;
    const int H = c.hidden;
    for (int i = 0; i < ns; ++i) {
        const Stream &st = r[i];
        QkvScatter q;
        memset(&q, 0, sizeof(q));
        q.qkv = m->qkv32; q.ld = 3 * H;
        q.qn_w = st.w->qn; q.kn_w = st.w->kn;
        q.rope_cs = st.rope_cs; q.rope = st.rope_cs != nullptr;
        q.q = m->q; q.k = m->k; q.vt = m->vt; q.ldv = m->ldv;
        q.seq = st.S; q.Ntot = Ntot; q.tok_off = st.tok_off;
        q.nh = c.n_head; q.rows = B * st.S;
        q.eps = QK_EPS;
        q.q_scale = Q_SCALE;
        q.v_rows = tuning().attn_vrows != 0;
        // Q8_0 weights: the scatter is the GEMM's epilogue (the same bits)
        const bool fused = st.w->qkv.type == TSK_TYPE_Q8_0 && tuning().q8_qkv_fused;
        int rc = g_lin(m, st.w->qkv, Rows{(const float *) st.xn, H, 0, 0}, B * st.S, m->qkv32, 3 * H, true, s,
                       fused ? &q : nullptr);
        if (rc) return rc;
        if (!fused && (rc = hipcheck(launch_qkv_scatter(q, s), "mmdit qkv scatter"))) return rc;
    }
    return TSK_OK;
}

int run_attention(tsk_mmdit *m, const Stream *r, int ns, int B, int Ntot, hipStream_t s) {
    const tsk_mmdit_config &c = m->cfg;
    AttnFastParams p;
    memset(&p, 0, sizeof(p));
    // bf16 rows for the fused path's BF16 linear1; F32 rows (the node's own
    // result, src/mmdit.cpp:91-93) otherwise
    const int es = m->fast ? 2 : 4;
    p.q = m->q; p.k = m->k; p.vt = m->vt; p.o = m->fast ? (void *) m->o : (void *) m->o32;
    p.q_type = TSK_TYPE_F16; p.k_bf16 = 0; p.out_bf16 = m->fast ? 1 : 0;
    p.Nq = p.Nkv = Ntot; p.H = c.n_head; p.B = B;
    p.q_nb1 = p.k_nb1 = 128;                          // q / k [B][n_head][Ntot][64] fp16
    p.q_nb2 = p.k_nb2 = (int64_t) 128 * Ntot;
    p.q_nb3 = p.k_nb3 = (int64_t) 128 * Ntot * c.n_head;
    p.vt_bh = (int64_t) 64 * m->ldv;
    p.ldv = m->ldv;
    p.o_nb1 = 64 * es; p.o_nb2 = (int64_t) es * c.hidden; p.o_nb3 = (int64_t) es * c.hidden * m->Nmax;
    p.c = Q_SCALE;
    p.q_prescaled = 1;
    float aq = 0.0f, ak = 0.0f;
    for (int i = 0; i < ns; ++i) {
        aq = fmaxf(aq, m->w[r[i].w->qn_idx].amax);
        ak = fmaxf(ak, m->w[r[i].w->kn_idx].amax);
    }
    // |q.k| <= 64 max|w_q| max|w_k| after RMSNorm (RoPE is a rotation): no
    // running max below ATTN_LOGIT_BOUND (1 % margin for the fp16 rounding)
    p.bounded = 1.01f * 64.0f * p.c * aq * ak <= ATTN_LOGIT_BOUND;
    p.force_cfg = tuning().attn_cfg;
    p.rule_b = m->cfg.max_batch;
    if (tuning().attn_vrows) {
        // the QKV epilogue or scatter wrote V as fp16 rows [B][n_head][Ntot][64] into vt
        p.v_rows = 1;
        p.v = m->vt;
        p.v_nb1 = 128; p.v_nb2 = (int64_t) 128 * Ntot; p.v_nb3 = (int64_t) 128 * Ntot * c.n_head;
    }
    return hipcheck(launch_attn_fast(p, s), "mmdit attention");
}

// post_attn (src/mmdit.cpp:226-235): linear1 on this stream's attention rows
// (its residual update is owed to the next LN), LN, ffn (owed to the next LN).
// The k3 convolutions of the latent and clip streams share their launches
// (two problems per GEMM); their partial sums and convMLP hidden states sit
// in separate slices.
int run_post(tsk_mmdit *m, Stream *r, int ns, int B, hipStream_t s) {
    const int H = m->cfg.hidden, F = m->cfg.mlp_hidden;
    const int64_t ob = (int64_t) m->Nmax * H;      // batch stride of the attention output rows
    int rc;
    GemmGroup gl;
    memset(&gl, 0, sizeof(gl));
    for (int i = 0; i < ns; ++i) {
        if (r[i].w->pre_only) continue;
        const Block &b = *r[i].w;
        const uint16_t *orows = m->o + (size_t) r[i].tok_off * H;
        if (b.conv) {
            r[i].pend_split = conv_splits(m, b.l1c, r[i].S);
            gl.p[gl.nprob++] = conv_problem(b.l1c, orows, H, ob, r[i].S, B, 1, r[i].part, H, true, r[i].pend_split);
        } else {
            // text: linear1 rows grouped by batch item
            GemmGroup g;
            memset(&g, 0, sizeof(g));
            g.nprob = 1;
            GemmProblem &q = g.p[0];
            q.x = orows; q.ld_x = H; q.x_group_rows = r[i].S; q.x_group_stride = ob;
            q.w = b.l1.w; q.ld_w = b.l1.K;
            q.y = r[i].part; q.ld_y = H;
            q.M = H; q.N = B * r[i].S; q.K = H; q.splits = 1;
            r[i].pend_split = 1;
            if ((rc = hipcheck(launch_gemm_coop(g, EPI_STORE_F32, s), "mmdit text linear1"))) return rc;
        }
        r[i].pending = true;
        r[i].pend_bias = b.conv ? b.l1c.b : b.l1.b;
        r[i].pend_gate = r[i].mod + 2 * H;             // gate_msa
        r[i].pend_ld = r[i].ld_mod;
    }
    // K slices (one when splits = 1) of both conv streams, no bias
    if (gl.nprob && (rc = hipcheck(launch_gemm_coop(gl, EPI_PARTIAL, s), "mmdit linear1 conv"))) return rc;
    Stream live[3];
    int nl = 0;
    for (int i = 0; i < ns; ++i)
        if (!r[i].w->pre_only) live[nl++] = r[i];
    if (!nl) return TSK_OK;
    if ((rc = run_ln(m, live, nl, B, 1, s))) return rc;
    GemmGroup g13, g2;
    memset(&g13, 0, sizeof(g13));
    memset(&g2, 0, sizeof(g2));
    int64_t hoff = 0;                                  // hidden-state slice of the next conv stream
    for (int i = 0, j = 0; i < ns; ++i) {
        if (r[i].w->pre_only) continue;
        r[i].pending = live[j++].pending;
        const Block &b = *r[i].w;
        if (b.conv) {
            uint16_t *hid = m->hid + hoff;
            hoff += (int64_t) B * r[i].S * F;
            GemmProblem &q = g13.p[g13.nprob++];
            q = conv_problem(b.w1c, (const uint16_t *) r[i].xn, H, (int64_t) r[i].S * H, r[i].S, B, 1, hid, F, true, 1);
            q.w3 = b.w3c.w;
            r[i].pend_split = conv_splits(m, b.w2c, r[i].S);
            g2.p[g2.nprob++] = conv_problem(b.w2c, hid, F, (int64_t) r[i].S * F, r[i].S, B, 1, r[i].part, H, true,
                                            r[i].pend_split);
        } else {
            r[i].pend_split = 1;
            if ((rc = lin_mlp(m, b.w1, b.w3, b.w2, (const uint16_t *) r[i].xn, H, B * r[i].S, r[i].part, H, s))) return rc;
        }
        r[i].pending = true;
        r[i].pend_bias = nullptr;
        r[i].pend_gate = r[i].mod + 5 * H;             // gate_mlp
        r[i].pend_ld = r[i].ld_mod;
    }
    if (g13.nprob) {
        // convmlp (src/mmdit.cpp:39-52): w2(silu(w1 x) * w3 x), the hidden state bf16
        if ((rc = hipcheck(launch_gemm_coop(g13, EPI_SWIGLU_BF16, s), "mmdit convmlp w1/w3"))) return rc;
        if ((rc = hipcheck(launch_gemm_coop(g2, EPI_PARTIAL, s), "mmdit convmlp w2"))) return rc;
    }
    return TSK_OK;
}

// post_attn on the f32 path, one stream after the other; each product's
// output is a whole (one-slice) partial sum that the next LN adds with bias
// and gate
int run_post_f32(tsk_mmdit *m, Stream *r, int ns, int B, hipStream_t s) {
    const int H = m->cfg.hidden;
    const int64_t ob = (int64_t) m->Nmax * H;
    int rc;
    for (int i = 0; i < ns; ++i) {
        if (r[i].w->pre_only) continue;
        const Block &b = *r[i].w;
        const float *orows = m->o32 + (size_t) r[i].tok_off * H;
        int sp = 1;
        if (b.conv) {
            sp = res_splits(m, b.l1c, r[i].S);
            rc = g_conv(m, b.l1c, orows, H, ob, r[i].S, B, 1, r[i].part, H, false, s, sp);
        } else {
            rc = g_lin(m, b.l1, Rows{orows, H, r[i].S, ob}, B * r[i].S, r[i].part, H, false, s);
        }
        if (rc) return rc;
        r[i].pending = true;
        r[i].pend_split = sp;
        r[i].pend_bias = b.conv ? b.l1c.b : b.l1.b;
        r[i].pend_gate = r[i].mod + 2 * H;             // gate_msa
        r[i].pend_ld = r[i].ld_mod;
    }
    Stream live[3];
    int nl = 0;
    for (int i = 0; i < ns; ++i)
        if (!r[i].w->pre_only) live[nl++] = r[i];
    if (!nl) return TSK_OK;
    if ((rc = run_ln(m, live, nl, B, 1, s))) return rc;
    for (int i = 0, j = 0; i < ns; ++i) {
        if (r[i].w->pre_only) continue;
        r[i].pending = live[j++].pending;
        const Block &b = *r[i].w;
        const float *xr = (const float *) r[i].xn;
        const int sp = b.conv ? res_splits(m, b.w2c, r[i].S) : 1;
        rc = g_swiglu(m, b.conv, b.w1c, b.w3c, b.w2c, b.w1, b.w3, b.w2, xr, H, (int64_t) r[i].S * H, r[i].S, B,
                      r[i].part, H, s, sp);
        if (rc) return rc;
        r[i].pending = true;
        r[i].pend_split = sp;
        r[i].pend_bias = nullptr;
        r[i].pend_gate = r[i].mod + 5 * H;             // gate_mlp
        r[i].pend_ld = r[i].ld_mod;
    }
    return TSK_OK;
}

}  // namespace

// ------------------------------------------------------------------ lifecycle
extern "C" void tsk_mmdit_default_config(tsk_mmdit_config *c) {
    if (!c) return;
    c->hidden = 1024; c->n_head = 16; c->head_dim = 64; c->depth = 21; c->fused_depth = 14;
    c->latent_dim = 64; c->text_seq = 77; c->clip_dim = 1024; c->sync_dim = 768; c->t5_dim = 2048;
    c->mlp_hidden = 2816; c->max_batch = 2; c->max_latent = 646; c->max_clip = 240; c->max_sync = 720;
    c->rope_theta = 10000.0f; c->t_max_period = 1.0f;
    c->weight_type = TSK_TYPE_BF16;
}

extern "C" void tsk_mmdit_destroy(tsk_mmdit *m) {
    if (!m) return;
    (void) hipDeviceSynchronize();
    void *bufs[] = {m->blob, m->lat, m->clip, m->txt, m->sync, m->ext, m->clip0, m->txt0, m->silu_ext, m->silu_gc,
                    m->vec, m->vec16, m->mods_lat, m->mods_gc, m->xn, m->hid, m->o, m->q, m->k, m->vt, m->part,
                    m->tmp32, m->rope_l, m->rope_c, m->in16, m->in32, m->act16, m->freq, m->temb, m->xn32, m->o32,
                    m->qkv32, m->hid32, m->h1, m->h3, m->cvt16, m->qx, m->dx, m->xs, m->f0, m->flow2};
    for (void *b : bufs)
        if (b) (void) hipFree(b);
    delete m;
}

namespace {

// type_of(weight) -> its storage type or a negative status
using TypeFn = std::function<int(const MW &)>;

int create_impl(const tsk_mmdit_config *cfg, const TypeFn &type_of, tsk_mmdit **out) {
    if (!out) return fail(TSK_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    int rc = validate_cfg(cfg);
    if (rc) return rc;
    if ((rc = require_init())) return rc;
    tsk_mmdit *m = new tsk_mmdit();
    m->cfg = *cfg;
    const tsk_mmdit_config &c = m->cfg;
    const int H = c.hidden, F = c.mlp_hidden, nj = c.depth - c.fused_depth, X = 2 * c.text_seq;
    // the converter's tensor names (convert/convert_thinksound.py:32) and shapes (docs/ARCHITECTURE.md §6.1)
    add_conv(m, "audio_input_proj.0", 3, c.latent_dim, H, true);
    add_conv(m, "audio_input_proj.2.w1", 3, H, F, false);
    add_conv(m, "audio_input_proj.2.w3", 3, H, F, false);
    add_conv(m, "audio_input_proj.2.w2", 3, F, H, false);
    add_lin(m, "clip_input_proj.0", c.clip_dim, H, true);
    add_conv(m, "clip_input_proj.2.w1", 3, H, F, false);
    add_conv(m, "clip_input_proj.2.w3", 3, H, F, false);
    add_conv(m, "clip_input_proj.2.w2", 3, F, H, false);
    add_conv(m, "sync_input_proj.0", 7, c.sync_dim, H, true);
    add_conv(m, "sync_input_proj.2.w1", 3, H, F, false);
    add_conv(m, "sync_input_proj.2.w3", 3, H, F, false);
    add_conv(m, "sync_input_proj.2.w2", 3, F, H, false);
    add_lin(m, "text_input_proj.0", c.t5_dim, H, true);
    add_lin(m, "text_input_proj.2.w1", H, F, false);
    add_lin(m, "text_input_proj.2.w3", H, F, false);
    add_lin(m, "text_input_proj.2.w2", F, H, false);
    add_lin(m, "text_cond_proj", c.clip_dim, H, true);
    add_lin(m, "clip_cond_proj", H, H, true);
    add_lin(m, "global_cond_mlp.w1", H, F, false);
    add_lin(m, "global_cond_mlp.w3", H, F, false);
    add_lin(m, "global_cond_mlp.w2", F, H, false);
    addw(m, "sync_pos_emb", c.sync_dim, 8, 1, K_VEC);
    add_lin(m, "t_embed.mlp.0", H, H, true);
    add_lin(m, "t_embed.mlp.2", H, H, true);
    for (int i = 0; i < nj; ++i) {
        const std::string p = "joint_blocks." + std::to_string(i);
        add_block(m, p + ".latent_block", false, true);
        add_block(m, p + ".clip_block", i == nj - 1, true);
        add_block(m, p + ".text_block", i == nj - 1, false);
    }
    for (int i = 0; i < c.fused_depth; ++i) add_block(m, "fused_blocks." + std::to_string(i), false, true);
    add_lin(m, "final_layer.adaLN_modulation.1", H, 2 * H, true);
    add_conv(m, "final_layer.conv", 7, H, c.latent_dim, true);
    addw(m, "empty_string_feat", c.clip_dim, c.text_seq, 1, K_VEC);
    addw(m, "empty_t5_feat", c.t5_dim, c.text_seq, 1, K_VEC);
    // storage types; the fused path needs every matrix BF16 but the t_embed MLP (F32)
    bool any_bf16 = false, any_q8 = false;
    for (MW &x : m->w) {
        const int t = type_of(x);
        if (t < 0) { tsk_mmdit_destroy(m); return t; }
        const bool ok = t == TSK_TYPE_F32 || (x.kind != K_VEC && t == TSK_TYPE_BF16) ||
                        (x.kind == K_LIN && t == TSK_TYPE_Q8_0 && x.ne[0] % 32 == 0);
        if (!ok) {
            tsk_mmdit_destroy(m);
            return fail(TSK_ERR_TYPE, "'%s': type %d is not supported for this tensor", x.name.c_str(), t);
        }
        x.type = t;
        any_bf16 = any_bf16 || t == TSK_TYPE_BF16;
        any_q8 = any_q8 || t == TSK_TYPE_Q8_0;
        m->fast = m->fast && t == rule_type(TSK_TYPE_BF16, x);
    }
    // F32 matrices also held as split bf16 planes (TSK_F32_SPLIT): every
    // linear and convolution of the f32 path but the adaLN sets (one GEMM
    // over a whole set) and the t_embed MLP (B rows, fp32 products)
    bool any_split = false;
    if (!m->fast && tuning().f32_split)
        for (MW &x : m->w) {
            x.split = x.type == TSK_TYPE_F32 && x.kind != K_VEC && x.name.find("adaLN_modulation") == std::string::npos &&
                      x.name.find("t_embed") == std::string::npos;
            any_split = any_split || x.split;
        }
    // blob placement: the adaLN weights (each plane of them), then biases, of
    // the latent blocks and the final layer back to back (rows of one [Ml][H]
    // matrix, 256-byte multiples: no gaps), the same for the clip and text
    // blocks, then every other tensor in inventory order; each set's adaLN is
    // one GEMM per forward
    std::vector<std::string> ada_l, ada_g;
    for (int i = 0; i < nj; ++i) ada_l.push_back("joint_blocks." + std::to_string(i) + ".latent_block");
    for (int i = 0; i < c.fused_depth; ++i) ada_l.push_back("fused_blocks." + std::to_string(i));
    ada_l.push_back("final_layer");
    for (int i = 0; i < nj; ++i) ada_g.push_back("joint_blocks." + std::to_string(i) + ".clip_block");
    for (int i = 0; i < nj; ++i) ada_g.push_back("joint_blocks." + std::to_string(i) + ".text_block");
    size_t off = 0;
    std::vector<int> placed(m->w.size(), 0);   // planes placed
    auto place = [&](const std::string &name, int plane) {
        const int i = m->idx.at(name);
        MW &x = m->w[i];
        const int64_t n = x.ne[0] * x.ne[1] * x.ne[2];
        const size_t bytes = plane == 2 ? (x.split ? 6 * (size_t) n : 0) : type_bytes(x.type, n, plane);
        if (!bytes) return;
        (plane == 2 ? x.offset_s : plane ? x.offset_d : x.offset) = off;
        off += (bytes + 255) & ~(size_t) 255;
        placed[i] |= 1 << plane;
    };
    for (const auto *set : {&ada_l, &ada_g}) {
        for (const auto &p : *set) place(p + ".adaLN_modulation.1.weight", 0);
        for (const auto &p : *set) place(p + ".adaLN_modulation.1.weight", 1);
        for (const auto &p : *set) place(p + ".adaLN_modulation.1.bias", 0);
    }
    for (size_t i = 0; i < m->w.size(); ++i)
        for (int plane = 0; plane < 3; ++plane)
            if (!(placed[i] & (1 << plane))) place(m->w[i].name, plane);
    const int B = c.max_batch, T = c.max_latent, C = c.max_clip, S = c.max_sync;
    const int64_t Ml = (int64_t) (nj + c.fused_depth) * 6 * H + 2 * H;          // latent blocks + final layer
    const int64_t Mg = (int64_t) 2 * (nj - 1) * 6 * H + 2 * 2 * H;             // clip + text (last pre_only)
    m->Nmax = T + C + X;
    m->ldv = (m->Nmax + 63) / 64 * 64;
    const int64_t R = (int64_t) B * std::max(std::max(T, C), std::max(S, X));   // rows of the longest stream
    m->Rmax = (int) R;
    const int64_t rows3 = (int64_t) B * (T + C + X);
    const int Wmax = std::max(std::max(H, c.t5_dim), std::max(c.sync_dim, c.clip_dim));
    const int Wcv = std::max(Wmax, F);                                          // widest product input
    // staged inputs per batch row: latent, clip, sync, text | t5, global text
    m->in_cap = (size_t) B * ((size_t) T * c.latent_dim + (size_t) C * c.clip_dim + (size_t) S * c.sync_dim +
                              (size_t) X * c.t5_dim + c.clip_dim);
    const size_t L = (size_t) c.latent_dim;
    auto alloc = [&](void **p, size_t bytes) -> int {
        hipError_t e = hipMalloc(p, bytes);
        if (e != hipSuccess) return fail(TSK_ERR_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return TSK_OK;
    };
    rc = TSK_OK;
    auto a = [&](void *p, size_t bytes) {
        if (!rc) rc = alloc((void **) p, bytes);
    };
    a(&m->blob, off);
    a(&m->lat, sizeof(float) * B * T * H);
    a(&m->clip, sizeof(float) * B * C * H);
    a(&m->txt, sizeof(float) * B * X * H);
    a(&m->clip0, sizeof(float) * B * C * H);
    a(&m->txt0, sizeof(float) * B * X * H);
    a(&m->sync, sizeof(float) * B * S * H);
    a(&m->ext, sizeof(float) * B * T * H);
    a(&m->vec, sizeof(float) * 8 * B * H);
    a(&m->mods_lat, sizeof(float) * B * T * Ml);
    a(&m->mods_gc, sizeof(float) * B * Mg);
    a(&m->q, 2 * (size_t) B * m->Nmax * H);
    a(&m->k, 2 * (size_t) B * m->Nmax * H);
    a(&m->vt, 2 * (size_t) B * H * m->ldv);
    a(&m->part, sizeof(float) * PART_SLICES * rows3 * H);
    a(&m->tmp32, sizeof(float) * R * std::max((size_t) H, L));
    a(&m->rope_l, sizeof(float) * T * 64);
    a(&m->rope_c, sizeof(float) * C * 64);
    a(&m->in32, sizeof(float) * m->in_cap);
    a(&m->freq, sizeof(float) * (H / 2));
    a(&m->temb, sizeof(float) * B * H);
    a(&m->xs, sizeof(float) * T * L);
    a(&m->f0, sizeof(float) * T * L);
    a(&m->flow2, sizeof(float) * std::max(B, 2) * T * L);
    if (m->fast) {
        a(&m->silu_ext, 2 * (size_t) B * T * H);
        a(&m->silu_gc, 2 * (size_t) B * H);
        a(&m->vec16, 2 * (size_t) 4 * B * Wmax);
        a(&m->xn, 2 * (size_t) rows3 * H);
        a(&m->hid, 2 * (size_t) std::max(R, (int64_t) B * (T + C)) * F);
        a(&m->o, 2 * (size_t) B * m->Nmax * H);
        a(&m->in16, 2 * m->in_cap);
        a(&m->act16, 2 * (size_t) R * H);
    } else {
        a(&m->xn32, sizeof(float) * rows3 * H);
        a(&m->o32, sizeof(float) * B * m->Nmax * H);
        a(&m->qkv32, sizeof(float) * R * 3 * H);
        a(&m->hid32, sizeof(float) * R * F);
        a(&m->h1, sizeof(float) * F32_KSPLIT_MAX * R * F);   // K-split slices of the F32 convMLP halves
        a(&m->h3, sizeof(float) * F32_KSPLIT_MAX * R * F);
        // conversions: at most R rows (B * T for the per-token adaLN) of the
        // widest input, three times as wide as split operands
        const size_t conv_rows = (size_t) std::max(R, (int64_t) B * T);
        if (any_bf16 || any_split) {
            m->cvt_cap = conv_rows * Wcv * (any_split ? 3 : 1);
            a(&m->cvt16, 2 * m->cvt_cap);
        }
        if (any_q8) {
            m->q_cap = conv_rows * Wcv;
            a(&m->qx, m->q_cap);
            a(&m->dx, sizeof(float) * (m->q_cap / 32));
        }
    }
    if (rc) { tsk_mmdit_destroy(m); return rc; }
    // t-embedding frequencies f_k = (1e4 / max_period) 1e4^(-2k / H) in host
    // fp32 as src/mmdit.cpp:309-311 evaluates them
    std::vector<float> fr(H / 2);
    for (int kk = 0; kk < H / 2; ++kk)
        fr[kk] = (10000.0f / c.t_max_period) * powf(10000.0f, -2.0f * (float) kk / (float) H);
    hipError_t e = hipMemcpy(m->freq, fr.data(), sizeof(float) * fr.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(m->blob, 0, off);
    // V^T key positions past a call's token count are read (times P = 0)
    if (e == hipSuccess) e = hipMemset(m->vt, 0, 2 * (size_t) B * H * m->ldv);
    // latent positions 0 .. T-1, freq_scale 1 (src/mmdit.cpp:96-99, :316-318)
    if (e == hipSuccess) e = launch_rope_table(m->rope_l, T, 64, powf(c.rope_theta, -2.0f / 64.0f), 1.0f, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) { tsk_mmdit_destroy(m); return hip_fail(e, "mmdit init"); }
    for (int i = 0; i < nj; ++i) {
        const std::string p = "joint_blocks." + std::to_string(i);
        m->jl.push_back(block_of(m, p + ".latent_block", false, true));
        m->jc.push_back(block_of(m, p + ".clip_block", i == nj - 1, true));
        m->jt.push_back(block_of(m, p + ".text_block", i == nj - 1, false));
    }
    for (int i = 0; i < c.fused_depth; ++i) m->fb.push_back(block_of(m, "fused_blocks." + std::to_string(i), false, true));
    // the two adaLN sets: columns in blob order (latent blocks, fused blocks,
    // final layer; clip blocks, text blocks)
    int64_t col = 0;
    for (auto &b : m->jl) { b.mod_col = col; col += (int64_t) b.nmod * H; }
    for (auto &b : m->fb) { b.mod_col = col; col += (int64_t) b.nmod * H; }
    m->fin_mod_col = col;
    col = 0;
    for (auto &b : m->jc) { b.mod_col = col; col += (int64_t) b.nmod * H; }
    for (auto &b : m->jt) { b.mod_col = col; col += (int64_t) b.nmod * H; }
    m->ada_lat = m->jl[0].ada;
    m->ada_lat.M = (int) Ml;
    m->ada_gc = m->jc[0].ada;
    m->ada_gc.M = (int) Mg;
    // every block's adaLN weight / scales / bias sits at its set's first
    // block's offset plus its first column's rows, in one type
    const Lin fin = lin_of(m, "final_layer.adaLN_modulation.1", true);
    auto at_col = [&](const Lin &base, const Lin &b, int64_t col0) {
        const int64_t rows = col0 * H;
        return b.type == base.type && b.b == base.b + col0 &&
               (b.type == TSK_TYPE_F32 ? b.wf == base.wf + rows
                : b.type == TSK_TYPE_BF16 ? b.w == base.w + rows
                                          : b.qw == base.qw + rows && b.dw == base.dw + rows / 32);
    };
    bool packed = at_col(m->ada_lat, fin, m->fin_mod_col);
    for (const auto *v : {&m->jl, &m->fb})
        for (const Block &b : *v) packed = packed && at_col(m->ada_lat, b.ada, b.mod_col);
    for (const auto *v : {&m->jc, &m->jt})
        for (const Block &b : *v) packed = packed && at_col(m->ada_gc, b.ada, b.mod_col);
    if (!packed) {
        tsk_mmdit_destroy(m);
        return fail(TSK_ERR_UNSUPPORTED, "every adaLN weight of a set must share one type");
    }
    m->h_pos_emb.assign((size_t) c.sync_dim * 8, 0.0f);
    m->h_empty_str.assign((size_t) c.clip_dim * c.text_seq, 0.0f);
    m->h_empty_t5.assign((size_t) c.t5_dim * c.text_seq, 0.0f);
    *out = m;
    return TSK_OK;
}

// host values in the driver's row order: qkv rows (h d j) -> [q | k | v]
// (rows of rowlen elements, or of rowlen blocks), conv kernels kw-major
std::vector<float> driver_order(const MW &x, int H, const float *src, int64_t n) {
    std::vector<float> v(src, src + n);
    if (x.qkv_perm) {
        const int64_t rowlen = x.kind == K_LIN ? x.ne[0] : 1;
        for (int64_t i = 0; i < H; ++i)
            for (int j = 0; j < 3; ++j)
                memcpy(&v[(size_t) ((j * H + i) * rowlen)], src + (3 * i + j) * rowlen, sizeof(float) * rowlen);
    }
    if (x.kind == K_CONV) {
        const int64_t KW = x.ne[0], IC = x.ne[1], OC = x.ne[2];
        std::vector<float> t((size_t) n);
        for (int64_t oc = 0; oc < OC; ++oc)
            for (int64_t ic = 0; ic < IC; ++ic)
                for (int64_t kw = 0; kw < KW; ++kw) t[(size_t) ((oc * KW + kw) * IC + ic)] = v[(size_t) ((oc * IC + ic) * KW + kw)];
        v.swap(t);
    }
    return v;
}

// Q8_0 blocks (rows already in the driver's order) -> the two planes on the device
int upload_q8(tsk_mmdit *m, const MW &x, const uint8_t *blocks) {
    const int64_t K = x.ne[0], M = x.ne[1];
    std::vector<int8_t> q((size_t) (M * K));
    std::vector<uint16_t> d((size_t) (M * K / 32));
    q8_blocks_to_planes(blocks, M, K, q.data(), d.data());
    hipError_t e = hipMemcpy(m->blob + x.offset, q.data(), q.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(m->blob + x.offset_d, d.data(), 2 * d.size(), hipMemcpyHostToDevice);
    return hipcheck(e, "mmdit q8_0 upload");
}

}  // namespace

extern "C" int tsk_mmdit_create(const tsk_mmdit_config *cfg, tsk_mmdit **out) {
    if (!cfg) return fail(TSK_ERR_INVALID_ARG, "cfg is NULL");
    const int wt = cfg->weight_type;
    return create_impl(cfg, [wt](const MW &x) { return rule_type(wt, x); }, out);
}

extern "C" int tsk_mmdit_n_tensors(const tsk_mmdit *m) { return m ? (int) m->w.size() : 0; }

extern "C" int tsk_mmdit_tensor_type(const tsk_mmdit *m, int i) {
    if (!m || i < 0 || i >= (int) m->w.size()) return fail(TSK_ERR_INVALID_ARG, "tensor index %d", i);
    return m->w[i].type;
}

extern "C" int tsk_mmdit_tensor_info(const tsk_mmdit *m, int i, const char **name, int64_t ne[4]) {
    if (!m || i < 0 || i >= (int) m->w.size()) return fail(TSK_ERR_INVALID_ARG, "tensor index %d", i);
    if (name) *name = m->w[i].name.c_str();
    if (ne) { ne[0] = m->w[i].ne[0]; ne[1] = m->w[i].ne[1]; ne[2] = m->w[i].ne[2]; ne[3] = 1; }
    return TSK_OK;
}

// host f32 in ggml / PyTorch memory order: linear [out][in], conv [OC][IC][KW]
// (ggml ne [KW, IC, OC]), vectors; held as the tensor's type: BF16 (RNE),
// F32, or Q8_0 (ggml's reference quantizer); conv kernels kw-major
// [OC][KW][IC], qkv rows (and bias entries) (h d j) -> [q | k | v]
extern "C" int tsk_mmdit_set_tensor(tsk_mmdit *m, const char *name, const float *src, int64_t n) {
    if (!m || !name || !src) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = m->idx.find(name);
    if (it == m->idx.end()) return fail(TSK_ERR_INVALID_ARG, "unknown tensor '%s'", name);
    MW &x = m->w[it->second];
    const int64_t N = x.ne[0] * x.ne[1] * x.ne[2];
    if (n != N) return fail(TSK_ERR_SHAPE, "'%s' has %lld elements, got %lld", name, (long long) N, (long long) n);
    const std::vector<float> v = driver_order(x, m->cfg.hidden, src, n);
    hipError_t e;
    if (x.kind == K_VEC) {
        float a = 0.0f;
        for (int64_t i = 0; i < n; ++i) a = fmaxf(a, fabsf(src[i]));
        x.amax = a;
        if (x.name == "sync_pos_emb") m->h_pos_emb.assign(src, src + n);
        if (x.name == "empty_string_feat") m->h_empty_str.assign(src, src + n);
        if (x.name == "empty_t5_feat") m->h_empty_t5.assign(src, src + n);
    }
    if (x.type == TSK_TYPE_F32) {
        e = hipMemcpy(m->blob + x.offset, v.data(), 4 * (size_t) n, hipMemcpyHostToDevice);
        if (e == hipSuccess && x.split) {
            // rows of K (a conv: KW groups of IC per output row) -> [hi | lo | hi]
            // per group, hi = bf16(w), lo = bf16(w - hi)
            const int64_t G = x.kind == K_CONV ? x.ne[1] : x.ne[0];
            std::vector<uint16_t> sp((size_t) (3 * n));
            for (int64_t g0 = 0; g0 < n; g0 += G)
                for (int64_t i = 0; i < G; ++i) {
                    const float w = v[(size_t) (g0 + i)];
                    const uint16_t hi = host_bf16_bits(w);
                    uint32_t hb = (uint32_t) hi << 16;
                    float hf;
                    memcpy(&hf, &hb, 4);
                    const uint16_t lo = std::isfinite(hf) ? host_bf16_bits(w - hf) : (uint16_t) 0;
                    uint16_t *d = &sp[(size_t) (3 * g0 + i)];
                    d[0] = hi;
                    d[G] = lo;
                    d[2 * G] = hi;
                }
            e = hipMemcpy(m->blob + x.offset_s, sp.data(), 2 * sp.size(), hipMemcpyHostToDevice);
        }
    } else if (x.type == TSK_TYPE_BF16) {
        std::vector<uint16_t> bf((size_t) n);
        for (int64_t i = 0; i < n; ++i) bf[i] = host_bf16_bits(v[i]);
        e = hipMemcpy(m->blob + x.offset, bf.data(), 2 * (size_t) n, hipMemcpyHostToDevice);
    } else {
        std::vector<uint8_t> blocks((size_t) (n / 32) * 34);
        q8_quantize_ref(v.data(), n / 32, blocks.data());
        return upload_q8(m, x, blocks.data());
    }
    return hipcheck(e, "mmdit set_tensor copy");
}

extern "C" int tsk_mmdit_set_tensor_q8_0(tsk_mmdit *m, const char *name, const void *blocks, size_t nbytes) {
    if (!m || !name || !blocks) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = m->idx.find(name);
    if (it == m->idx.end()) return fail(TSK_ERR_INVALID_ARG, "unknown tensor '%s'", name);
    const MW &x = m->w[it->second];
    if (x.type != TSK_TYPE_Q8_0) return fail(TSK_ERR_TYPE, "'%s' is not held as Q8_0 by this model", name);
    const size_t rowbytes = (size_t) (x.ne[0] / 32) * 34;
    if (nbytes != rowbytes * (size_t) x.ne[1])
        return fail(TSK_ERR_SHAPE, "'%s' has %zu bytes of Q8_0 blocks, got %zu", name, rowbytes * (size_t) x.ne[1], nbytes);
    if (!x.qkv_perm) return upload_q8(m, x, (const uint8_t *) blocks);
    // whole rows of blocks: source row 3 i + j -> row j H + i
    const int H = m->cfg.hidden;
    std::vector<uint8_t> pb(nbytes);
    for (int64_t i = 0; i < H; ++i)
        for (int j = 0; j < 3; ++j)
            memcpy(&pb[(size_t) (j * H + i) * rowbytes], (const uint8_t *) blocks + (size_t) (3 * i + j) * rowbytes,
                   rowbytes);
    return upload_q8(m, x, pb.data());
}

// ------------------------------------------------------------------ forward
namespace {

int check_fwd(const tsk_mmdit *m, int B, int T, int clip_S, int sync_S) {
    const tsk_mmdit_config &c = m->cfg;
    if (B < 1 || B > c.max_batch) return fail(TSK_ERR_SHAPE, "B=%d outside [1, %d]", B, c.max_batch);
    if (T < 1 || T > c.max_latent) return fail(TSK_ERR_SHAPE, "T=%d outside [1, %d]", T, c.max_latent);
    if (clip_S < 1 || clip_S > c.max_clip) return fail(TSK_ERR_SHAPE, "clip_S=%d outside [1, %d]", clip_S, c.max_clip);
    if (sync_S < 8 || sync_S > c.max_sync || sync_S % 8)
        return fail(TSK_ERR_SHAPE, "sync_S=%d must be a multiple of 8 in [8, %d]", sync_S, c.max_sync);
    return require_init();
}

// the inputs of one forward: HOST rows (one pointer per batch row, each in
// ts_dit::forward's layout) or DEVICE arrays with the batch outermost; t on
// the host either way. latent may be null (the sampler stages it itself).
struct Inputs {
    bool device;
    const float *const *latent, *const *clip, *const *sync, *const *text, *const *t5, *const *g;
    const float *d_latent, *d_clip, *d_sync, *d_text, *d_t5, *d_g;
};

// one call's shapes and its regions of the f32 (and bf16) staging areas:
// latent rows [B][T][L], clip [B][clip_S][clip_dim], sync (+ pos_emb)
// [B][sync_S][sync_dim], text_f zero-padded to t5_dim and t5 along the
// sequence [B][2 text_seq][t5_dim], global text [B][clip_dim]
struct Call {
    int B, T, clip_S, sync_S;
    size_t n_lat, n_cond;
    float *lat, *clip, *sync, *txt, *g;
    const uint16_t *lat16, *clip16, *sync16, *txt16, *g16;
};

int make_call(tsk_mmdit *m, int B, int T, int clip_S, int sync_S, Call &k) {
    const tsk_mmdit_config &c = m->cfg;
    const int X = 2 * c.text_seq;
    k.B = B; k.T = T; k.clip_S = clip_S; k.sync_S = sync_S;
    const size_t n_clip = (size_t) B * clip_S * c.clip_dim, n_sync = (size_t) B * sync_S * c.sync_dim,
                 n_txt = (size_t) B * X * c.t5_dim, n_g = (size_t) B * c.clip_dim;
    k.n_lat = (size_t) B * T * c.latent_dim;
    k.n_cond = n_clip + n_sync + n_txt + n_g;
    if (k.n_lat + k.n_cond > m->in_cap) return fail(TSK_ERR_SHAPE, "staged inputs exceed the capacity");
    k.lat = m->in32;
    k.clip = k.lat + k.n_lat; k.sync = k.clip + n_clip; k.txt = k.sync + n_sync; k.g = k.txt + n_txt;
    k.lat16 = k.clip16 = k.sync16 = k.txt16 = k.g16 = nullptr;
    if (m->in16) {   // the fused path's bf16 copies, at the same offsets
        k.lat16 = m->in16; k.clip16 = k.lat16 + k.n_lat; k.sync16 = k.clip16 + n_clip; k.txt16 = k.sync16 + n_sync;
        k.g16 = k.txt16 + n_txt;
    }
    return TSK_OK;
}

// the conditioning inputs (and the latent, when given) into the staging
// area: the latent transposed to rows (the ggml_transpose of :151), sync +
// per-segment pos_emb (:169-172), text_f zero-padded to t5_dim concatenated
// with t5 (:179-180). The host path keeps its pageable source alive until
// the stream has consumed it.
int stage_inputs(tsk_mmdit *m, const Call &k, const Inputs &in, hipStream_t st) {
    const tsk_mmdit_config &c = m->cfg;
    const int B = k.B, T = k.T, L = c.latent_dim, X = 2 * c.text_seq;
    const bool with_lat = in.device ? in.d_latent != nullptr : in.latent != nullptr;
    if (!in.device) {
        const size_t n_all = k.n_lat + k.n_cond;
        std::vector<float> hs(n_all, 0.0f);
        float *h_lat = hs.data(), *h_clip = h_lat + k.n_lat, *h_sync = h_clip + (k.sync - k.clip),
              *h_txt = h_sync + (k.txt - k.sync), *h_g = h_txt + (k.g - k.txt);
        for (int b = 0; b < B; ++b) {
            if (with_lat)
                for (int ch = 0; ch < L; ++ch)
                    for (int t = 0; t < T; ++t) h_lat[((size_t) b * T + t) * L + ch] = in.latent[b][(size_t) ch * T + t];
            memcpy(h_clip + (size_t) b * k.clip_S * c.clip_dim, in.clip[b], sizeof(float) * k.clip_S * c.clip_dim);
            for (int s = 0; s < k.sync_S; ++s)
                for (int ch = 0; ch < c.sync_dim; ++ch)
                    h_sync[((size_t) b * k.sync_S + s) * c.sync_dim + ch] =
                        in.sync[b][(size_t) s * c.sync_dim + ch] + m->h_pos_emb[(size_t) (s % 8) * c.sync_dim + ch];
            for (int s = 0; s < c.text_seq; ++s) {
                memcpy(h_txt + ((size_t) b * X + s) * c.t5_dim, in.text[b] + (size_t) s * c.clip_dim,
                       sizeof(float) * c.clip_dim);
                memcpy(h_txt + ((size_t) b * X + c.text_seq + s) * c.t5_dim, in.t5[b] + (size_t) s * c.t5_dim,
                       sizeof(float) * c.t5_dim);
            }
            memcpy(h_g + (size_t) b * c.clip_dim, in.g[b], sizeof(float) * c.clip_dim);
        }
        const size_t skip = with_lat ? 0 : k.n_lat;
        hipError_t e = hipMemcpyAsync(k.lat + skip, hs.data() + skip, sizeof(float) * (n_all - skip),
                                      hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        return hipcheck(e, "inputs");
    }
    const float *pe = wp<float>(m, "sync_pos_emb");
    hipError_t e = hipSuccess;
    if (with_lat) e = launch_transpose_ct(in.d_latent, B, L, T, k.lat, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(k.clip, in.d_clip, sizeof(float) * B * k.clip_S * c.clip_dim, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = launch_add_period_rows(in.d_sync, (int64_t) B * k.sync_S, c.sync_dim, pe, 8, k.sync, st);
    if (e == hipSuccess) e = hipMemsetAsync(k.txt, 0, sizeof(float) * B * X * c.t5_dim, st);
    for (int b = 0; b < B && e == hipSuccess; ++b) {
        e = hipMemcpy2DAsync(k.txt + (size_t) b * X * c.t5_dim, sizeof(float) * c.t5_dim,
                             in.d_text + (size_t) b * c.text_seq * c.clip_dim, sizeof(float) * c.clip_dim,
                             sizeof(float) * c.clip_dim, c.text_seq, hipMemcpyDeviceToDevice, st);
        if (e == hipSuccess)
            e = hipMemcpyAsync(k.txt + ((size_t) b * X + c.text_seq) * c.t5_dim, in.d_t5 + (size_t) b * c.text_seq * c.t5_dim,
                               sizeof(float) * c.text_seq * c.t5_dim, hipMemcpyDeviceToDevice, st);
    }
    if (e == hipSuccess) e = hipMemcpyAsync(k.g, in.d_g, sizeof(float) * B * c.clip_dim, hipMemcpyDeviceToDevice, st);
    return hipcheck(e, "device inputs");
}

// vector slots of m->vec ([8][B][H])
enum Vec { V_TE0 = 0, V_TE, V_TFC, V_CMEAN, V_CFC, V_GSUM, V_GCM, V_GC };
float *vslot(tsk_mmdit *m, int B, int i) { return m->vec + (size_t) i * B * m->cfg.hidden; }

// The conditioning that does not depend on t (src/mmdit.cpp:163-193): clip
// -> clip0, sync, text -> txt0, global_cond_mlp(clip_cond(mean clip) +
// text_cond(g)) -> the gcmlp slot, and the clip RoPE table.
int prep_cond(tsk_mmdit *m, const Call &k, hipStream_t st) {
    const tsk_mmdit_config &c = m->cfg;
    const int H = c.hidden, X = 2 * c.text_seq, B = k.B;
    float *tfc = vslot(m, B, V_TFC), *cmean = vslot(m, B, V_CMEAN), *cfc = vslot(m, B, V_CFC),
          *gsum = vslot(m, B, V_GSUM), *gcm = vslot(m, B, V_GCM);
    int rc;
    if (m->fast) {
        // bf16 copies of the staged conditioning inputs (the BF16 mul_mats round their src1)
        if ((rc = hipcheck(launch_f32_to_bf16(k.clip, (uint16_t *) k.clip16, (int64_t) k.n_cond, st), "inputs bf16")))
            return rc;
        uint16_t *v16 = m->vec16, *a16 = m->act16;
        // clip: linear -> silu -> convMLP (:163-167)
        if ((rc = lin(lin_of(m, "clip_input_proj.0", true), k.clip16, c.clip_dim, B * k.clip_S, m->tmp32, H, false, st)) ||
            (rc = hipcheck(launch_silu_bf16(m->tmp32, a16, (int64_t) B * k.clip_S * H, st), "silu")) ||
            (rc = conv_mlp(m, conv_of(m, "clip_input_proj.2.w1", false), conv_of(m, "clip_input_proj.2.w3", false),
                           conv_of(m, "clip_input_proj.2.w2", false), a16, H, (int64_t) k.clip_S * H, k.clip_S, B,
                           m->clip0, H, st)))
            return rc;
        // sync: conv k7 (padding 3) -> silu -> convMLP (:168-177)
        if ((rc = conv_plain(m, conv_of(m, "sync_input_proj.0", true), k.sync16, c.sync_dim,
                             (int64_t) k.sync_S * c.sync_dim, k.sync_S, B, 3, m->tmp32, H, true, st)) ||
            (rc = hipcheck(launch_silu_bf16(m->tmp32, a16, (int64_t) B * k.sync_S * H, st), "silu")) ||
            (rc = conv_mlp(m, conv_of(m, "sync_input_proj.2.w1", false), conv_of(m, "sync_input_proj.2.w3", false),
                           conv_of(m, "sync_input_proj.2.w2", false), a16, H, (int64_t) k.sync_S * H, k.sync_S, B,
                           m->sync, H, st)))
            return rc;
        // text: linear (t5_dim -> H) -> silu -> MLP (:179-183)
        if ((rc = lin(lin_of(m, "text_input_proj.0", true), k.txt16, c.t5_dim, B * X, m->tmp32, H, false, st)) ||
            (rc = hipcheck(launch_silu_bf16(m->tmp32, a16, (int64_t) B * X * H, st), "silu")) ||
            (rc = lin_mlp(m, lin_of(m, "text_input_proj.2.w1", false), lin_of(m, "text_input_proj.2.w3", false),
                          lin_of(m, "text_input_proj.2.w2", false), a16, H, B * X, m->txt0, H, st)))
            return rc;
        // conditioning vectors (:184-193)
        if ((rc = lin(lin_of(m, "text_cond_proj", true), k.g16, c.clip_dim, B, tfc, H, false, st)) ||
            (rc = hipcheck(launch_row_mean(m->clip0, B, k.clip_S, H, cmean, st), "clip mean")) ||
            (rc = hipcheck(launch_f32_to_bf16(cmean, v16, (int64_t) B * H, st), "bf16")) ||
            (rc = lin(lin_of(m, "clip_cond_proj", true), v16, H, B, cfc, H, false, st)) ||
            (rc = hipcheck(launch_add_f32(cfc, tfc, gsum, (int64_t) B * H, st), "add")) ||
            (rc = hipcheck(launch_f32_to_bf16(gsum, v16, (int64_t) B * H, st), "bf16")) ||
            (rc = lin_mlp(m, lin_of(m, "global_cond_mlp.w1", false), lin_of(m, "global_cond_mlp.w3", false),
                          lin_of(m, "global_cond_mlp.w2", false), v16, H, B, gcm, H, st)))
            return rc;
    } else {
        float *t32 = m->tmp32;
        if ((rc = g_lin(m, lin_of(m, "clip_input_proj.0", true), Rows{k.clip, c.clip_dim, 0, 0}, B * k.clip_S, t32, H,
                        true, st)) ||
            (rc = hipcheck(launch_silu_inplace(t32, (int64_t) B * k.clip_S * H, st), "silu")) ||
            (rc = g_conv_mlp(m, "clip_input_proj.2", t32, H, (int64_t) k.clip_S * H, k.clip_S, B, m->clip0, H, st)))
            return rc;
        if ((rc = g_conv(m, conv_of(m, "sync_input_proj.0", true), k.sync, c.sync_dim, (int64_t) k.sync_S * c.sync_dim,
                         k.sync_S, B, 3, t32, H, true, st)) ||
            (rc = hipcheck(launch_silu_inplace(t32, (int64_t) B * k.sync_S * H, st), "silu")) ||
            (rc = g_conv_mlp(m, "sync_input_proj.2", t32, H, (int64_t) k.sync_S * H, k.sync_S, B, m->sync, H, st)))
            return rc;
        if ((rc = g_lin(m, lin_of(m, "text_input_proj.0", true), Rows{k.txt, c.t5_dim, 0, 0}, B * X, t32, H, true,
                        st)) ||
            (rc = hipcheck(launch_silu_inplace(t32, (int64_t) B * X * H, st), "silu")) ||
            (rc = g_lin_mlp(m, "text_input_proj.2", t32, H, B * X, m->txt0, H, st)))
            return rc;
        if ((rc = g_lin(m, lin_of(m, "text_cond_proj", true), Rows{k.g, c.clip_dim, 0, 0}, B, tfc, H, true, st)) ||
            (rc = hipcheck(launch_row_mean(m->clip0, B, k.clip_S, H, cmean, st), "clip mean")) ||
            (rc = g_lin(m, lin_of(m, "clip_cond_proj", true), Rows{cmean, H, 0, 0}, B, cfc, H, true, st)) ||
            (rc = hipcheck(launch_add_f32(cfc, tfc, gsum, (int64_t) B * H, st), "add")) ||
            (rc = g_lin_mlp(m, "global_cond_mlp", gsum, H, B, gcm, H, st)))
            return rc;
    }
    if ((rc = grab(m, "clip_pp", m->clip0, (size_t) B * k.clip_S * H, st)) ||
        (rc = grab(m, "text_pp", m->txt0, (size_t) B * X * H, st)) ||
        (rc = grab(m, "clip_fc", cfc, (size_t) B * H, st)) || (rc = grab(m, "text_fc", tfc, (size_t) B * H, st)) ||
        (rc = grab(m, "gcmlp", gcm, (size_t) B * H, st)))
        return rc;
    // clip RoPE: positions 0 .. clip_S - 1, freq_scale T / clip_S (:237, :318)
    return hipcheck(launch_rope_table(m->rope_c, k.clip_S, 64, powf(c.rope_theta, -2.0f / 64.0f),
                                      (float) k.T / (float) k.clip_S, st),
                    "clip rope table");
}

// One flow evaluation after prep_cond on the same call shapes: the staged
// latent rows (k.lat) and one t per batch row -> flow rows [B][T][L] (device)
int step(tsk_mmdit *m, const Call &k, const float *t, float *flow, hipStream_t st) {
    const tsk_mmdit_config &c = m->cfg;
    const int H = c.hidden, L = c.latent_dim, X = 2 * c.text_seq, nj = c.depth - c.fused_depth;
    const int B = k.B, T = k.T, clip_S = k.clip_S;
    const int Ntot = T + clip_S + X;
    int rc;
    float *te0 = vslot(m, B, V_TE0), *te = vslot(m, B, V_TE), *gcm = vslot(m, B, V_GCM), *gc = vslot(m, B, V_GC);
    // ---- audio_input_proj: conv k3 -> silu -> convMLP (:150-155)
    if (m->fast) {
        if ((rc = hipcheck(launch_f32_to_bf16(k.lat, (uint16_t *) k.lat16, (int64_t) k.n_lat, st), "latent bf16")) ||
            (rc = conv(conv_of(m, "audio_input_proj.0", true), k.lat16, L, (int64_t) T * L, T, B, 1, m->tmp32, H, false,
                       st)) ||
            (rc = hipcheck(launch_silu_bf16(m->tmp32, m->act16, (int64_t) B * T * H, st), "silu")) ||
            (rc = conv_mlp(m, conv_of(m, "audio_input_proj.2.w1", false), conv_of(m, "audio_input_proj.2.w3", false),
                           conv_of(m, "audio_input_proj.2.w2", false), m->act16, H, (int64_t) T * H, T, B, m->lat, H,
                           st)))
            return rc;
    } else {
        if ((rc = g_conv(m, conv_of(m, "audio_input_proj.0", true), k.lat, L, (int64_t) T * L, T, B, 1, m->tmp32, H,
                         true, st)) ||
            (rc = hipcheck(launch_silu_inplace(m->tmp32, (int64_t) B * T * H, st), "silu")) ||
            (rc = g_conv_mlp(m, "audio_input_proj.2", m->tmp32, H, (int64_t) T * H, T, B, m->lat, H, st)))
            return rc;
    }
    if ((rc = grab(m, "x_in", m->lat, (size_t) B * T * H, st))) return rc;
    // ---- timestep embedding [cos(t f_k), sin(t f_k)] (:305-314; f_k from the
    // host formula) -> t_embed MLP (:157-161)
    TimeVals tv;
    memset(&tv, 0, sizeof(tv));
    for (int b = 0; b < B; ++b) tv.t[b] = t[b];
    if ((rc = hipcheck(launch_timestep_embed(m->freq, tv, B, H, m->temb, st), "timestep embedding"))) return rc;
    const Lin te_a = lin_of(m, "t_embed.mlp.0", true), te_b = lin_of(m, "t_embed.mlp.2", true);
    if (te_a.type == TSK_TYPE_F32) rc = lin_f32(te_a, m->temb, B, te0, st);
    else rc = g_lin(m, te_a, Rows{m->temb, H, 0, 0}, B, te0, H, true, st);
    if (rc || (rc = hipcheck(launch_silu_inplace(te0, (int64_t) B * H, st), "silu"))) return rc;
    if (te_b.type == TSK_TYPE_F32) rc = lin_f32(te_b, te0, B, te, st);
    else rc = g_lin(m, te_b, Rows{te0, H, 0, 0}, B, te, H, true, st);
    if (rc || (rc = grab(m, "t_emb", te, (size_t) B * H, st))) return rc;
    // ---- global_c = gcmlp + t_emb, extended_c (:194-196)
    if ((rc = hipcheck(launch_add_f32(gcm, te, gc, (int64_t) B * H, st), "add")) ||
        (rc = hipcheck(launch_sync_extend(m->sync, B, k.sync_S, T, H, gc, m->ext, st), "extended_c")) ||
        (rc = grab(m, "global_c", gc, (size_t) B * H, st)) ||
        (rc = grab(m, "extended_c", m->ext, (size_t) B * T * H, st)))
        return rc;
    // every block's adaLN (lin(adaLN, silu(c)), :209) in two GEMMs: per token
    // from extended_c (latent blocks, final layer), per item from global_c
    // (clip and text blocks); each output is the same dot product a per-block
    // launch computes
    const int64_t Ml = m->ada_lat.M, Mg = m->ada_gc.M;
    if (m->fast) {
        if ((rc = hipcheck(launch_silu_bf16(m->ext, m->silu_ext, (int64_t) B * T * H, st), "silu")) ||
            (rc = hipcheck(launch_silu_bf16(gc, m->silu_gc, (int64_t) B * H, st), "silu")) ||
            (rc = lin(m->ada_lat, m->silu_ext, H, B * T, m->mods_lat, Ml, false, st)) ||
            (rc = lin(m->ada_gc, m->silu_gc, H, B, m->mods_gc, Mg, false, st)))
            return rc;
    } else {
        // silu in place: extended_c and global_c are not read again this step
        if ((rc = hipcheck(launch_silu_inplace(m->ext, (int64_t) B * T * H, st), "silu")) ||
            (rc = hipcheck(launch_silu_inplace(gc, (int64_t) B * H, st), "silu")) ||
            (rc = g_lin(m, m->ada_lat, Rows{m->ext, H, 0, 0}, B * T, m->mods_lat, Ml, true, st)) ||
            (rc = g_lin(m, m->ada_gc, Rows{gc, H, 0, 0}, B, m->mods_gc, Mg, true, st)))
            return rc;
    }
    // the clip and text streams start from their input projections
    hipError_t e = hipMemcpyAsync(m->clip, m->clip0, sizeof(float) * B * clip_S * H, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(m->txt, m->txt0, sizeof(float) * B * X * H, hipMemcpyDeviceToDevice, st);
    if ((rc = hipcheck(e, "stream copies"))) return rc;

    // ---- joint blocks over latent | clip | text (:238-271)
    const size_t rL = 0, rC = (size_t) B * T, rX = rC + (size_t) B * clip_S;   // stream rows in xn / part
    const size_t es = m->fast ? 2 : 4;
    char *xnb = m->fast ? (char *) m->xn : (char *) m->xn32;
    Stream Ls, Cs, Xs;
    memset(&Ls, 0, sizeof(Ls));
    memset(&Cs, 0, sizeof(Cs));
    memset(&Xs, 0, sizeof(Xs));
    Ls.x = m->lat; Ls.S = T; Ls.tok_off = 0; Ls.rope_cs = m->rope_l; Ls.per_token = 1;
    Ls.xn = xnb + es * rL * H; Ls.part = m->part + PART_SLICES * rL * H;
    Cs.x = m->clip; Cs.S = clip_S; Cs.tok_off = T; Cs.rope_cs = m->rope_c; Cs.per_token = 0;
    Cs.xn = xnb + es * rC * H; Cs.part = m->part + PART_SLICES * rC * H;
    Xs.x = m->txt; Xs.S = X; Xs.tok_off = T + clip_S; Xs.rope_cs = nullptr; Xs.per_token = 0;
    Xs.xn = xnb + es * rX * H; Xs.part = m->part + PART_SLICES * rX * H;
    // a block's residual updates are applied by the next LayerNorm launch:
    // the stage tensors after block 0 and after the joint blocks are taken
    // right after that launch
    bool cap_jb0 = false, cap_joint = false;
    auto capture = [&]() -> int {
        int r = TSK_OK;
        if (cap_jb0) {
            cap_jb0 = false;
            if ((r = grab(m, "jb0_lat", m->lat, (size_t) B * T * H, st)) ||
                (r = grab(m, "jb0_clip", m->clip, (size_t) B * clip_S * H, st)) ||
                (r = grab(m, "jb0_text", m->txt, (size_t) B * X * H, st)))
                return r;
        }
        if (cap_joint) {
            cap_joint = false;
            r = grab(m, "after_joint", m->lat, (size_t) B * T * H, st);
        }
        return r;
    };
    auto qkv = m->fast ? run_qkv : run_qkv_f32;
    auto post = m->fast ? run_post : run_post_f32;
    for (int i = 0; i < nj; ++i) {
        Ls.w = &m->jl[i];
        Cs.w = &m->jc[i];
        Xs.w = &m->jt[i];
        Ls.mod = m->mods_lat + Ls.w->mod_col; Ls.ld_mod = Ml;
        Cs.mod = m->mods_gc + Cs.w->mod_col; Cs.ld_mod = Mg;
        Xs.mod = m->mods_gc + Xs.w->mod_col; Xs.ld_mod = Mg;
        Stream r3[3] = {Ls, Cs, Xs};
        if ((rc = run_ln(m, r3, 3, B, 0, st)) || (rc = capture())) return rc;
        if ((rc = qkv(m, r3, 3, B, Ntot, st))) return rc;
        if ((rc = run_attention(m, r3, 3, B, Ntot, st))) return rc;
        if ((rc = post(m, r3, 3, B, st))) return rc;
        Ls = r3[0];
        Cs = r3[1];
        Xs = r3[2];
        cap_jb0 = i == 0;
    }
    cap_joint = true;
    // ---- fused blocks on the latent with extended_c (:274-281)
    for (int i = 0; i < c.fused_depth; ++i) {
        Ls.w = &m->fb[i];
        Ls.mod = m->mods_lat + Ls.w->mod_col; Ls.ld_mod = Ml;
        if ((rc = run_ln(m, &Ls, 1, B, 0, st)) || (rc = capture())) return rc;
        if ((rc = qkv(m, &Ls, 1, B, T, st))) return rc;
        if ((rc = run_attention(m, &Ls, 1, B, T, st))) return rc;
        if ((rc = post(m, &Ls, 1, B, st))) return rc;
    }
    // ---- final layer: adaLN(extended_c) -> LN / modulate -> conv k7 (:284-289)
    Block fin;
    memset(&fin, 0, sizeof(fin));
    fin.nmod = 2;
    fin.ada = lin_of(m, "final_layer.adaLN_modulation.1", true);
    Ls.w = &fin;
    Ls.mod = m->mods_lat + m->fin_mod_col; Ls.ld_mod = Ml;
    if ((rc = run_ln(m, &Ls, 1, B, 0, st)) || (rc = capture())) return rc;
    if ((rc = grab(m, "after_fused", m->lat, (size_t) B * T * H, st))) return rc;
    const Conv fc = conv_of(m, "final_layer.conv", true);
    if (m->fast) return conv_plain(m, fc, (const uint16_t *) Ls.xn, H, (int64_t) T * H, T, B, 3, flow, L, true, st);
    return g_conv(m, fc, (const float *) Ls.xn, H, (int64_t) T * H, T, B, 3, flow, L, true, st);
}

// flow: per-row HOST outputs (host inputs; the call synchronises) or one
// DEVICE array [B][T][latent_dim] (device inputs; no host synchronisation)
int forward_impl(tsk_mmdit *m, int B, int T, int clip_S, int sync_S, const Inputs &in, const float *t,
                 float *const *flow, float *d_flow, hipStream_t st) {
    Call k;
    int rc = make_call(m, B, T, clip_S, sync_S, k);
    if (rc) return rc;
    m->stages.clear();
    if ((rc = stage_inputs(m, k, in, st)) || (rc = prep_cond(m, k, st))) return rc;
    float *f = in.device ? d_flow : m->flow2;
    if ((rc = step(m, k, t, f, st))) return rc;
    if (in.device) return TSK_OK;
    const int L = m->cfg.latent_dim;
    std::vector<float> hf((size_t) B * T * L);
    hipError_t e = hipMemcpyAsync(hf.data(), f, sizeof(float) * hf.size(), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if ((rc = hipcheck(e, "flow"))) return rc;
    for (int b = 0; b < B; ++b) memcpy(flow[b], hf.data() + (size_t) b * T * L, sizeof(float) * T * L);
    return TSK_OK;
}

}  // namespace

extern "C" int tsk_mmdit_forward(tsk_mmdit *m, int B, int T, const float *latent, const float *t, int clip_S,
                                 const float *clip_f, int sync_S, const float *sync_f, const float *text_f,
                                 const float *t5, const float *global_text, float *flow, tsk_stream stream) {
    if (!m || !latent || !t || !clip_f || !sync_f || !text_f || !t5 || !global_text || !flow)
        return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    int rc = check_fwd(m, B, T, clip_S, sync_S);
    if (rc) return rc;
    const tsk_mmdit_config &c = m->cfg;
    std::vector<const float *> pl(B), pc(B), ps(B), px(B), p5(B), pg(B);
    std::vector<float *> pf(B);
    for (int b = 0; b < B; ++b) {
        pl[b] = latent + (size_t) b * c.latent_dim * T;
        pc[b] = clip_f + (size_t) b * clip_S * c.clip_dim;
        ps[b] = sync_f + (size_t) b * sync_S * c.sync_dim;
        px[b] = text_f + (size_t) b * c.text_seq * c.clip_dim;
        p5[b] = t5 + (size_t) b * c.text_seq * c.t5_dim;
        pg[b] = global_text + (size_t) b * c.clip_dim;
        pf[b] = flow + (size_t) b * T * c.latent_dim;
    }
    Inputs in{false, pl.data(), pc.data(), ps.data(), px.data(), p5.data(), pg.data(),
              nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    return forward_impl(m, B, T, clip_S, sync_S, in, t, pf.data(), nullptr, (hipStream_t) stream);
}

extern "C" int tsk_mmdit_forward_device(tsk_mmdit *m, int B, int T, const float *latent_d, const float *t,
                                        int clip_S, const float *clip_d, int sync_S, const float *sync_d,
                                        const float *text_d, const float *t5_d, const float *global_text_d,
                                        float *flow_d, tsk_stream stream) {
    if (!m || !latent_d || !t || !clip_d || !sync_d || !text_d || !t5_d || !global_text_d || !flow_d)
        return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    int rc = check_fwd(m, B, T, clip_S, sync_S);
    if (rc) return rc;
    Inputs in{true, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
              latent_d, clip_d, sync_d, text_d, t5_d, global_text_d};
    return forward_impl(m, B, T, clip_S, sync_S, in, t, nullptr, flow_d, (hipStream_t) stream);
}

extern "C" int tsk_mmdit_debug(tsk_mmdit *m, int enable) {
    if (!m) return fail(TSK_ERR_INVALID_ARG, "m is NULL");
    m->debug = enable != 0;
    if (!m->debug) m->stages.clear();
    return TSK_OK;
}

extern "C" int64_t tsk_mmdit_debug_size(const tsk_mmdit *m, const char *name) {
    if (!m || !name) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = m->stages.find(name);
    return it == m->stages.end() ? (int64_t) fail(TSK_ERR_INVALID_ARG, "no stage '%s'", name) : (int64_t) it->second.size();
}

extern "C" int tsk_mmdit_debug_get(const tsk_mmdit *m, const char *name, float *out, int64_t n) {
    if (!m || !name || !out) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = m->stages.find(name);
    if (it == m->stages.end()) return fail(TSK_ERR_INVALID_ARG, "no stage '%s'", name);
    if ((size_t) n != it->second.size()) return fail(TSK_ERR_SHAPE, "stage '%s' has %zu values", name, it->second.size());
    memcpy(out, it->second.data(), sizeof(float) * (size_t) n);
    return TSK_OK;
}

// ts_dit::sample (src/mmdit.cpp:344-376): per step one forward of B = 2 rows,
// row 0 conditional, row 1 unconditional (the learned empty_string_feat /
// empty_t5_feat and a zero global text feature, :350-357). The conditioning
// that does not depend on t is computed once; x stays on the device, and
// v = u + cfg (c - u), x += dt v run after each step's forward in the
// reference's order and rounding (cfg_euler), which also writes the next
// step's two latent rows.
extern "C" int tsk_mmdit_sample(tsk_mmdit *m, int T, const float *noise, int clip_S, const float *clip_f, int sync_S,
                                const float *sync_f, const float *text_f, const float *t5, const float *global_text,
                                int steps, float cfg_scale, float *out, float *flow0, tsk_stream stream) {
    if (!m || !noise || !clip_f || !sync_f || !text_f || !t5 || !global_text || !out)
        return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    if (m->cfg.max_batch < 2) return fail(TSK_ERR_SHAPE, "CFG needs max_batch >= 2");
    if (steps < 1) return fail(TSK_ERR_INVALID_ARG, "steps=%d", steps);
    int rc = check_fwd(m, 2, T, clip_S, sync_S);
    if (rc) return rc;
    hipStream_t st = (hipStream_t) stream;
    const tsk_mmdit_config &c = m->cfg;
    const int L = c.latent_dim;
    const size_t n = (size_t) T * L;
    Call k;
    if ((rc = make_call(m, 2, T, clip_S, sync_S, k))) return rc;
    m->stages.clear();
    const std::vector<float> zeros((size_t) c.clip_dim, 0.0f);
    const float *pc[2] = {clip_f, clip_f}, *ps[2] = {sync_f, sync_f};
    const float *px[2] = {text_f, m->h_empty_str.data()}, *p5[2] = {t5, m->h_empty_t5.data()},
                *pg[2] = {global_text, zeros.data()};
    Inputs in{false, nullptr, pc, ps, px, p5, pg, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    if ((rc = stage_inputs(m, k, in, st)) || (rc = prep_cond(m, k, st))) return rc;
    // noise ne = [T, L] -> token-major x [T][L], and both latent rows of the first step
    std::vector<float> hx(n);
    for (int ch = 0; ch < L; ++ch)
        for (int t = 0; t < T; ++t) hx[(size_t) t * L + ch] = noise[(size_t) ch * T + t];
    hipError_t e = hipMemcpyAsync(m->xs, hx.data(), sizeof(float) * n, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(k.lat, m->xs, sizeof(float) * n, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(k.lat + n, m->xs, sizeof(float) * n, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if ((rc = hipcheck(e, "noise"))) return rc;
    for (int s = 0; s < steps; ++s) {
        const float t_curr = 1.0f - (float) s / (float) steps;
        const float t_prev = 1.0f - (float) (s + 1) / (float) steps;
        const float dt = t_prev - t_curr;
        const float tt[2] = {t_curr, t_curr};
        if ((rc = step(m, k, tt, m->flow2, st))) return rc;
        if ((rc = hipcheck(launch_cfg_euler(m->flow2, (int64_t) n, cfg_scale, dt, m->xs, k.lat, s == 0 ? m->f0 : nullptr,
                                            st),
                           "cfg / euler")))
            return rc;
    }
    std::vector<float> hf(flow0 ? n : 0);
    e = hipMemcpyAsync(hx.data(), m->xs, sizeof(float) * n, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess && flow0) e = hipMemcpyAsync(hf.data(), m->f0, sizeof(float) * n, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if ((rc = hipcheck(e, "sample result"))) return rc;
    for (int ch = 0; ch < L; ++ch)
        for (int t = 0; t < T; ++t) {
            out[(size_t) ch * T + t] = hx[(size_t) t * L + ch];
            if (flow0) flow0[(size_t) ch * T + t] = hf[(size_t) t * L + ch];
        }
    return TSK_OK;
}

// ------------------------------------------------------------------ GGUF (ts_dit::load)
namespace {

// a metadata value when the file has the key (absent keys keep *dst)
void gguf_u32(const tsk_gguf *g, const char *key, int *dst) {
    uint32_t v;
    if (tsk_gguf_get_u32(g, key, &v) == TSK_OK) *dst = (int) v;
}

void gguf_f32(const tsk_gguf *g, const char *key, float *dst) {
    float v;
    if (tsk_gguf_get_f32(g, key, &v) == TSK_OK) *dst = v;
}

}  // namespace

// ts_dit::load (src/mmdit.cpp:104-116): the model sizes from the dit.* keys
// convert/convert_thinksound.py:38-45 writes (absent keys keep the values in
// *cfg), the SwiGLU width from audio_input_proj.2.w1 ([3, hidden, width]),
// and a weight_type that names the file's matrices (Q8_0 if any is Q8_0,
// else the type of the first qkv projection). Capacities are the caller's.
extern "C" int tsk_mmdit_config_from_gguf(const tsk_gguf *g, tsk_mmdit_config *c) {
    if (!g || !c) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    gguf_u32(g, "dit.hidden_dim", &c->hidden);
    gguf_u32(g, "dit.depth", &c->depth);
    gguf_u32(g, "dit.fused_depth", &c->fused_depth);
    gguf_u32(g, "dit.num_heads", &c->n_head);
    gguf_u32(g, "dit.latent_dim", &c->latent_dim);
    gguf_u32(g, "dit.text_seq_len", &c->text_seq);
    gguf_u32(g, "dit.clip_dim", &c->clip_dim);
    gguf_u32(g, "dit.sync_dim", &c->sync_dim);
    gguf_u32(g, "dit.text_dim", &c->t5_dim);
    gguf_f32(g, "dit.rope_theta", &c->rope_theta);
    gguf_f32(g, "dit.t_embed_max_period", &c->t_max_period);
    if (c->n_head > 0) c->head_dim = c->hidden / c->n_head;
    int64_t ne[4];
    int type;
    if (tsk_gguf_find_tensor(g, "audio_input_proj.2.w1.weight", ne, &type) >= 0) c->mlp_hidden = (int) ne[2];
    bool q8 = false;
    for (int i = 0; i < tsk_gguf_n_tensors(g); ++i) {
        const char *nm;
        if (tsk_gguf_tensor_info(g, i, &nm, ne, &type) == TSK_OK && type == TSK_TYPE_Q8_0) q8 = true;
    }
    if (q8) c->weight_type = TSK_TYPE_Q8_0;
    else if (tsk_gguf_find_tensor(g, "joint_blocks.0.latent_block.attn.qkv.weight", ne, &type) >= 0)
        c->weight_type = type == TSK_TYPE_F32 ? TSK_TYPE_F32 : TSK_TYPE_BF16;
    return TSK_OK;
}

// every weight by name (ts_model::load_backend, src/common/ts_model.cpp:13-41):
// Q8_0 blocks bit for bit, F32 / BF16 / F16 values exactly (into F32 or
// BF16 storage of the same values); a tensor whose file type the model does
// not hold it in is refused
extern "C" int tsk_mmdit_load_gguf(tsk_mmdit *m, const tsk_gguf *g) {
    if (!m || !g) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    std::vector<float> buf;
    std::vector<uint8_t> raw;
    for (const MW &x : m->w) {
        int64_t ne[4];
        int type;
        if (tsk_gguf_find_tensor(g, x.name.c_str(), ne, &type) < 0)
            return fail(TSK_ERR_INVALID_ARG, "GGUF file has no tensor '%s'", x.name.c_str());
        const int64_t n = x.ne[0] * x.ne[1] * x.ne[2];
        if (ne[0] * ne[1] * ne[2] * ne[3] != n || ne[0] != x.ne[0])
            return fail(TSK_ERR_SHAPE, "GGUF tensor '%s' is [%lld, %lld, %lld], the model needs [%lld, %lld, %lld]",
                        x.name.c_str(), (long long) ne[0], (long long) ne[1], (long long) (ne[2] * ne[3]),
                        (long long) x.ne[0], (long long) x.ne[1], (long long) x.ne[2]);
        int rc;
        if (type == TSK_TYPE_Q8_0 || x.type == TSK_TYPE_Q8_0) {
            if (type != x.type)
                return fail(TSK_ERR_TYPE, "GGUF tensor '%s' has type %d, the model holds it as type %d", x.name.c_str(),
                            type, x.type);
            raw.resize((size_t) (n / 32) * 34);
            if ((rc = tsk_gguf_read_tensor(g, x.name.c_str(), 0, raw.data(), raw.size())) ||
                (rc = tsk_mmdit_set_tensor_q8_0(m, x.name.c_str(), raw.data(), raw.size())))
                return rc;
            continue;
        }
        // a BF16 model holds F32 / F16 file matrices only when their values are
        // bf16 values; an F32 model holds every float type exactly
        if (x.kind != K_VEC && x.type == TSK_TYPE_BF16 && type != TSK_TYPE_BF16)
            return fail(TSK_ERR_TYPE, "GGUF tensor '%s' has type %d, the model holds it as BF16", x.name.c_str(), type);
        buf.resize((size_t) n);
        if ((rc = tsk_gguf_read_tensor(g, x.name.c_str(), 1, buf.data(), buf.size() * 4)) ||
            (rc = tsk_mmdit_set_tensor(m, x.name.c_str(), buf.data(), n)))
            return rc;
    }
    return TSK_OK;
}

// a model holding every tensor in its file's type, then loaded
extern "C" int tsk_mmdit_create_from_gguf(const tsk_gguf *g, const tsk_mmdit_config *cfg, tsk_mmdit **out) {
    if (!g || !cfg || !out) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto type_of = [g](const MW &x) -> int {
        int64_t ne[4];
        int type;
        if (tsk_gguf_find_tensor(g, x.name.c_str(), ne, &type) < 0)
            return fail(TSK_ERR_INVALID_ARG, "GGUF file has no tensor '%s'", x.name.c_str());
        if (x.kind == K_VEC) return TSK_TYPE_F32;
        if (type == TSK_TYPE_F16) return fail(TSK_ERR_TYPE, "'%s': F16 matrices are not supported", x.name.c_str());
        return type;
    };
    int rc = create_impl(cfg, type_of, out);
    if (rc) return rc;
    if ((rc = tsk_mmdit_load_gguf(*out, g))) {
        tsk_mmdit_destroy(*out);
        *out = nullptr;
    }
    return rc;
}
