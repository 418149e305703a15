// dit.cpp — MM-DiT flow-step driver and CFG sampler on gfx950 (counterpart of
// ts_dit, src/mmdit.h:9-42 / src/mmdit.cpp:119-376).
//
// One forward() runs, for B batch rows (CFG cond/uncond as B = 2):
//   host: t-embedding frequencies (mmdit.cpp:305-314), uploaded;
//   t_embed MLP (:158-160) -> silu(cond);
//   ONE launch for every block's adaLN GEMV (they only depend on cond);
//   input projection; 7 joint blocks (latent + text streams, the last text
//   stream pre_only, :238-271) and 14 fused blocks (:275-281), each:
//     LN+modulate -> QKV GEMM -> split/RMSNorm/RoPE into the attention
//     layout -> flash attention over the concatenated tokens ->
//     out-proj GEMM with fused gate*residual -> LN+modulate ->
//     fc1 GEMM with fused GELU -> fc2 GEMM with fused gate*residual;
//   final adaLN/LN/modulate + output projection (:285-289).
// Weights are stored once as bf16 (matrices) / f32 (biases, norm weights);
// the QKV rows are permuted from the reference's interleaved (h d j) order
// (split_qkv, mmdit.cpp:67-76) to [q | k | v] blocks at load, which is exact.
// Activations live in preallocated device buffers sized for max_batch x
// max_latent; nothing is allocated per forward.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/tsk/tsk.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

using namespace tsk;

namespace {

struct WInfo {
    std::string name;
    int64_t ne0, ne1;      // ggml ne: [in, out] for matrices, [n] for vectors
    bool matrix;           // stored bf16
    bool qkv_perm;         // rows (or entries) permuted (h d j) -> [q | k | v]
    bool tiled;            // stored in the MFMA-tiled layout of the block GEMMs
    bool q8;               // stored as Q8_0 planes: int8 [ne1][ne0], fp16 d [ne1][ne0 / 32]
    size_t offset;         // bytes into the weight blob
    float amax;            // max |value| of a vector as last set (0 until then)
};

struct RoleTiming {
    std::vector<hipEvent_t> ev;   // start/stop pairs, reused across resets
    size_t used = 0;
    int64_t launches = 0;
    double flop = 0.0, bytes = 0.0;
};

// split-K slices of the two K-reducing block projections; fixed, so every
// output element is summed in the same order whatever the batch or length
constexpr int KSPLIT_MAX = 4;    // split-K slices of linear1 (default 2) / ffn.fc2 (default 4), Tuning

struct Q8W {                // a Q8_0 matrix as planes
    const int8_t *q;
    const uint16_t *d;
};

struct StreamW {           // one MMDitSingleBlock's weights
    const uint16_t *ada_w, *qkv_w, *l1_w, *fc1_w, *fc2_w;
    Q8W qkv_q, l1_q, fc1_q, fc2_q;   // the Q8_0 driver's block projections
    const float *ada_b, *qkv_b, *qn, *kn, *l1_b, *fc1_b, *fc2_b;
    bool pre_only;
    float *mod;            // [max_batch][nmod * H] adaLN output
    int nmod;
    size_t sched_off;      // offset of this block's modulations in a schedule row
    int qn_idx, kn_idx;    // tensor indices of the q / k RMSNorm weights
};

}  // namespace

struct tsk_dit {
    tsk_dit_config cfg;
    std::vector<WInfo> w;
    std::unordered_map<std::string, int> idx;
    char *blob = nullptr;
    size_t blob_bytes = 0;
    std::vector<StreamW> joint_lat, joint_txt, fused;
    // activations
    float *lat = nullptr, *txt = nullptr, *flow = nullptr, *xf = nullptr;
    float *in_stage = nullptr;      // tsk_dit_forward's device copies of the host latent and text
    float *temb = nullptr, *tmp_c = nullptr, *cvec = nullptr;
    float *mods = nullptr;
    float *final_mod = nullptr;     // [max_batch][2H] final-layer adaLN output
    // sampler conditioning schedule: every step's adaLN outputs, one row of
    // sched_row floats per step (blocks at StreamW::sched_off, final layer at
    // sched_final), computed in one batched pass before the first step
    float *sched = nullptr;
    size_t sched_cap = 0, sched_row = 0, sched_final = 0;
    float *sched_act = nullptr;       // [3][32][H]: temb, t_embed hidden, silu(cond) of 32 steps
    GemvJob *sched_jobs = nullptr;    // device job tables, one per 32-step chunk
    int sched_jobs_cap = 0;
    std::vector<GemvJob> jobs_host;   // the adaLN job table (blocks, final layer, t_embed.0, .2)
    std::vector<size_t> jobs_sched_off;   // schedule-row offset of each adaLN job's output
    const float *cur_sched = nullptr; // the schedule row of the running step (nullptr: computed per call)
    // bf16 activations: xn [rows][H] (LN outputs), h [rows][F] (GELU outputs),
    // latent rows first, text rows from the fixed offset max_batch * max_latent;
    // fp16 attention operands q/k [B][n_head][Ntot][64], V transposed
    // vt [B][n_head][64][ldv] (key positions vt_pos()); o bf16 [B][Ntot][H]
    uint16_t *xn = nullptr, *q = nullptr, *k = nullptr, *vt = nullptr, *o = nullptr, *h = nullptr;
    int ldv = 0;
    float *part = nullptr;          // split-K partial sums [KSPLIT_MAX][rows][H], text at the same offset rule
    GemvJob *jobs_dev = nullptr;    // [adaLN jobs..., t_embed.0, t_embed.2]
    int njobs = 0, max_job_m = 0;
    float *freq = nullptr;          // t-embedding frequencies [H/2] (host formula)
    float *rope_cs = nullptr;       // RoPE (cos, sin) [max_latent][head_dim] of the latent positions
    // block GEMM tile shape per projection (qkv, out, fc1, fc2): a launch_gemm_ks
    // cfg, or 0 for the shape rule of gemm_cfg_for() (Tuning::gemm_cfg overrides)
    int gemm_cfg[4] = {0, 0, 0, 0};
    int ksplit_out = 2, ksplit_fc2 = 4;
    bool ksplit_auto = true;        // linear1's split-K by latent tokens (ksplit_out_for)
    bool timing = false;
    int attn_cfg = 0;               // attention launch shape override (0: automatic)
    // second stream for the adaLN GEMVs of the later blocks (HBM-bound) while
    // the first blocks compute; fork / join events
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    RoleTiming rt[TSK_ROLE_COUNT];
    // sampler buffers
    float *s_x = nullptr, *s_x2 = nullptr, *s_text2 = nullptr, *s_flow2 = nullptr, *s_flow0 = nullptr;
    // Q8_0 driver (weight_type Q8_0): f32 QKV rows [rows][3 H], f32 attention
    // output [B][Ntot][H], f32 GELU outputs [rows][F], and the Q8_0 planes of
    // the activations a block projection reads (int8 qx [rows][<= F], f32
    // block scales dx [rows][<= F / 32]); latent rows first, text rows from
    // the capacity offset
    bool q8 = false;
    float *qkv32 = nullptr, *o32 = nullptr, *dx = nullptr, *dh = nullptr;
    int8_t *qx = nullptr, *qh = nullptr;   // qh / dh: the GELU output of fc1 as Q8_0 planes (fc2's input)
};

namespace {

int hipcheck(hipError_t e, const char *what) { return e == hipSuccess ? TSK_OK : hip_fail(e, what); }

// Makes the launches in its lifetime stamp an event pair with their own
// execution start / end (launch_kernel) when the driver's timing is enabled,
// and books their algorithmic FLOPs / bytes.
struct Timed {
    RoleTiming *r = nullptr;
    hipEvent_t stop = nullptr;
    hipStream_t st;
    Timed(tsk_dit *d, int role, double flop, double bytes, hipStream_t s) : st(s) {
        if (!d->timing) return;
        r = &d->rt[role];
        if (r->used + 2 > r->ev.size()) {
            hipEvent_t a, b;
            if (hipEventCreate(&a) != hipSuccess) { r = nullptr; return; }
            if (hipEventCreate(&b) != hipSuccess) { (void) hipEventDestroy(a); r = nullptr; return; }
            r->ev.push_back(a);
            r->ev.push_back(b);
        }
        hipEvent_t start = r->ev[r->used];
        stop = r->ev[r->used + 1];
        r->used += 2;
        r->launches += 1;
        r->flop += flop;
        r->bytes += bytes;
        launch_events() = LaunchEvents{start, stop};
    }
    ~Timed() {
        if (r) launch_events() = LaunchEvents{nullptr, nullptr};
    }
};

void add(tsk_dit *d, const std::string &name, int64_t ne0, int64_t ne1, bool matrix, bool perm = false,
         bool tiled = false) {
    WInfo wi;
    wi.name = name;
    wi.ne0 = ne0;
    wi.ne1 = ne1;
    wi.matrix = matrix;
    wi.qkv_perm = perm;
    // the block projections (the tiled matrices) are Q8_0 in the Q8_0 driver
    wi.q8 = tiled && d->cfg.weight_type == TSK_TYPE_Q8_0;
    wi.tiled = tiled && !wi.q8;
    wi.offset = 0;
    wi.amax = 0.0f;
    d->idx[name] = (int) d->w.size();
    d->w.push_back(wi);
}

void add_block(tsk_dit *d, const std::string &p, bool pre_only) {
    const int H = d->cfg.hidden, F = d->cfg.mlp_hidden, hd = d->cfg.head_dim;
    const int nmod = pre_only ? 2 : 6;
    add(d, p + ".adaLN_modulation.1.weight", H, nmod * H, true);
    add(d, p + ".adaLN_modulation.1.bias", nmod * H, 1, false);
    add(d, p + ".attn.qkv.weight", H, 3 * H, true, true, true);
    add(d, p + ".attn.qkv.bias", 3 * H, 1, false, true);
    add(d, p + ".attn.q_norm.weight", hd, 1, false);
    add(d, p + ".attn.k_norm.weight", hd, 1, false);
    if (!pre_only) {
        add(d, p + ".linear1.weight", H, H, true, false, true);
        add(d, p + ".linear1.bias", H, 1, false);
        add(d, p + ".ffn.fc1.weight", H, F, true, false, true);
        add(d, p + ".ffn.fc1.bias", F, 1, false);
        add(d, p + ".ffn.fc2.weight", F, H, true, false, true);
        add(d, p + ".ffn.fc2.bias", H, 1, false);
    }
}

template <class T> T *wptr(tsk_dit *d, const std::string &name) {
    return (T *) (d->blob + d->w[d->idx.at(name)].offset);
}

StreamW stream_weights(tsk_dit *d, const std::string &p, bool pre_only) {
    StreamW s;
    memset(&s, 0, sizeof(s));
    s.pre_only = pre_only;
    s.nmod = pre_only ? 2 : 6;
    s.ada_w = wptr<uint16_t>(d, p + ".adaLN_modulation.1.weight");
    s.ada_b = wptr<float>(d, p + ".adaLN_modulation.1.bias");
    s.qkv_w = wptr<uint16_t>(d, p + ".attn.qkv.weight");
    s.qkv_b = wptr<float>(d, p + ".attn.qkv.bias");
    s.qn = wptr<float>(d, p + ".attn.q_norm.weight");
    s.kn = wptr<float>(d, p + ".attn.k_norm.weight");
    s.qn_idx = d->idx.at(p + ".attn.q_norm.weight");
    s.kn_idx = d->idx.at(p + ".attn.k_norm.weight");
    auto q8w = [&](const std::string &name) {
        const WInfo &wi = d->w[d->idx.at(name)];
        Q8W r{nullptr, nullptr};
        if (wi.q8) {
            r.q = (const int8_t *) (d->blob + wi.offset);
            r.d = (const uint16_t *) (d->blob + wi.offset + (size_t) (wi.ne0 * wi.ne1));
        }
        return r;
    };
    s.qkv_q = q8w(p + ".attn.qkv.weight");
    if (!pre_only) {
        s.l1_q = q8w(p + ".linear1.weight");
        s.fc1_q = q8w(p + ".ffn.fc1.weight");
        s.fc2_q = q8w(p + ".ffn.fc2.weight");
    }
    if (!pre_only) {
        s.l1_w = wptr<uint16_t>(d, p + ".linear1.weight");
        s.l1_b = wptr<float>(d, p + ".linear1.bias");
        s.fc1_w = wptr<uint16_t>(d, p + ".ffn.fc1.weight");
        s.fc1_b = wptr<float>(d, p + ".ffn.fc1.bias");
        s.fc2_w = wptr<uint16_t>(d, p + ".ffn.fc2.weight");
        s.fc2_b = wptr<float>(d, p + ".ffn.fc2.bias");
    }
    return s;
}

int validate_cfg(const tsk_dit_config *c) {
    if (!c) return fail(TSK_ERR_INVALID_ARG, "cfg is NULL");
    if (c->head_dim != 64) return fail(TSK_ERR_UNSUPPORTED, "head_dim must be 64");
    if (c->hidden != c->n_head * c->head_dim) return fail(TSK_ERR_SHAPE, "hidden != n_head * head_dim");
    if (c->n_head < 1 || c->n_head > 64) return fail(TSK_ERR_SHAPE, "n_head %d", c->n_head);
    if (c->depth < c->fused_depth || c->depth - c->fused_depth < 1 || c->fused_depth < 0)
        return fail(TSK_ERR_SHAPE, "depth %d / fused_depth %d", c->depth, c->fused_depth);
    if (c->mlp_kind != TSK_MLP_GELU_TANH) return fail(TSK_ERR_UNSUPPORTED, "mlp_kind %d", c->mlp_kind);
    if (c->weight_type != TSK_TYPE_BF16 && c->weight_type != TSK_TYPE_Q8_0)
        return fail(TSK_ERR_UNSUPPORTED, "DiT weights must be BF16 or Q8_0");
    if (c->weight_type == TSK_TYPE_Q8_0 && ((c->hidden != 1024 && c->hidden != 2048) || c->mlp_hidden % 128))
        return fail(TSK_ERR_UNSUPPORTED, "the Q8_0 driver needs hidden 1024 or 2048 and mlp_hidden %% 128 == 0");
    if (c->mlp_hidden % 64 || c->latent_dim % 8 || c->latent_dim < 8 || c->latent_dim > c->hidden || c->text_seq < 1)
        return fail(TSK_ERR_SHAPE, "mlp_hidden %% 64, latent_dim %% 8 and <= hidden");
    if (c->max_batch < 1 || c->max_batch > 32 || c->max_latent < 1) return fail(TSK_ERR_SHAPE, "capacity");
    if (!(c->ln_eps > 0) || !(c->qk_eps > 0) || !(c->rope_theta > 0) || !(c->t_max_period > 0))
        return fail(TSK_ERR_INVALID_ARG, "eps / theta / period");
    return TSK_OK;
}

}  // namespace

// ------------------------------------------------------------------ config / lifecycle
extern "C" void tsk_dit_default_config(tsk_dit_config *c) {
    if (!c) return;
    c->hidden = 1024; c->n_head = 16; c->head_dim = 64; c->depth = 21; c->fused_depth = 14;
    c->latent_dim = 64; c->text_seq = 77; c->mlp_hidden = 4096; c->mlp_kind = TSK_MLP_GELU_TANH;
    c->weight_type = TSK_TYPE_BF16; c->max_batch = 2; c->max_latent = 646;
    c->rope_theta = 10000.0f; c->t_max_period = 1.0f; c->ln_eps = 1e-5f; c->qk_eps = 1e-6f;
}

extern "C" void tsk_dit_destroy(tsk_dit *d) {
    if (!d) return;
    (void) hipDeviceSynchronize();
    for (auto &r : d->rt)
        for (hipEvent_t e : r.ev) (void) hipEventDestroy(e);
    if (d->ev_fork) (void) hipEventDestroy(d->ev_fork);
    if (d->ev_join) (void) hipEventDestroy(d->ev_join);
    if (d->side) (void) hipStreamDestroy(d->side);
    void *bufs[] = {d->sched, d->sched_act, d->sched_jobs,
                    d->blob, d->lat, d->txt, d->flow, d->in_stage, d->xf, d->temb, d->tmp_c, d->cvec, d->mods,
                    d->xn, d->part,
                    d->q, d->k, d->vt, d->o, d->h, d->jobs_dev, d->freq, d->rope_cs,
                    d->s_x /* one allocation: s_x2, s_flow2, s_flow0, s_text2 point into it */,
                    d->qkv32, d->o32, d->qh, d->dh, d->qx, d->dx};
    for (void *b : bufs)
        if (b) (void) hipFree(b);
    delete d;
}

extern "C" int tsk_dit_create(const tsk_dit_config *cfg, tsk_dit **out) {
    if (!out) return fail(TSK_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    int rc = validate_cfg(cfg);
    if (rc) return rc;
    if ((rc = require_init())) return rc;
    tsk_dit *d = new tsk_dit();
    d->cfg = *cfg;
    // launch-shape overrides of tuning sweeps (attention shape, block GEMM
    // tiles per projection), fixed at create
    d->attn_cfg = tuning().attn_cfg;
    for (int i = 0; i < 4; ++i) d->gemm_cfg[i] = tuning().gemm_cfg[i];
    d->ksplit_out = tuning().ksplit_out;
    d->ksplit_auto = !tuning().ksplit_set;
    d->ksplit_fc2 = tuning().ksplit_fc2;
    const tsk_dit_config &c = d->cfg;
    const int H = c.hidden, nj = c.depth - c.fused_depth;
    add(d, "audio_input_proj.weight", c.latent_dim, H, true);
    add(d, "audio_input_proj.bias", H, 1, false);
    add(d, "t_embed.mlp.0.weight", H, H, true);
    add(d, "t_embed.mlp.0.bias", H, 1, false);
    add(d, "t_embed.mlp.2.weight", H, H, true);
    add(d, "t_embed.mlp.2.bias", H, 1, false);
    for (int i = 0; i < nj; ++i) {
        add_block(d, "joint_blocks." + std::to_string(i) + ".latent_block", false);
        add_block(d, "joint_blocks." + std::to_string(i) + ".text_block", i == nj - 1);
    }
    for (int i = 0; i < c.fused_depth; ++i) add_block(d, "fused_blocks." + std::to_string(i), false);
    add(d, "final_layer.adaLN_modulation.1.weight", H, 2 * H, true);
    add(d, "final_layer.adaLN_modulation.1.bias", 2 * H, 1, false);
    add(d, "final_layer.linear.weight", H, c.latent_dim, true);
    add(d, "final_layer.linear.bias", c.latent_dim, 1, false);
    size_t off = 0;
    for (auto &wi : d->w) {
        wi.offset = off;
        const size_t bytes = wi.q8 ? tsk_q8_0_split_nbytes(wi.ne0, wi.ne1) : (size_t) (wi.ne0 * wi.ne1) * (wi.matrix ? 2 : 4);
        off += (bytes + 255) & ~(size_t) 255;
    }
    d->blob_bytes = off;

    const int B = c.max_batch, T = c.max_latent, St = c.text_seq, F = c.mlp_hidden;
    const int64_t rows = (int64_t) B * (T + St);
    d->ldv = (T + St + 63) / 64 * 64;
    auto alloc = [&](void **p, size_t bytes) -> int {
        hipError_t e = hipMalloc(p, bytes);
        if (e != hipSuccess) return fail(TSK_ERR_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return TSK_OK;
    };
    // adaLN outputs: one region per stream block + final layer
    size_t mod_floats = 0;
    const int nstreams = 2 * nj + c.fused_depth;
    mod_floats = (size_t) B * 6 * H * nstreams + (size_t) B * 2 * H;
    if ((rc = alloc((void **) &d->blob, d->blob_bytes)) ||
        (rc = alloc((void **) &d->lat, sizeof(float) * B * T * H)) ||
        (rc = alloc((void **) &d->txt, sizeof(float) * B * St * H)) ||
        (rc = alloc((void **) &d->flow, sizeof(float) * B * T * c.latent_dim)) ||
        (rc = alloc((void **) &d->in_stage, sizeof(float) * B * ((size_t) T * c.latent_dim + (size_t) c.text_seq * H))) ||
        (rc = alloc((void **) &d->xf, sizeof(float) * B * T * H)) ||
        (rc = alloc((void **) &d->temb, sizeof(float) * B * H)) ||
        (rc = alloc((void **) &d->tmp_c, sizeof(float) * B * H)) ||
        (rc = alloc((void **) &d->cvec, sizeof(float) * B * H)) ||
        (rc = alloc((void **) &d->mods, sizeof(float) * mod_floats)) ||
        (rc = alloc((void **) &d->xn, 2 * rows * H)) ||
        (rc = alloc((void **) &d->part, sizeof(float) * KSPLIT_MAX * rows * H)) ||
        (rc = alloc((void **) &d->q, 2 * rows * H)) ||
        (rc = alloc((void **) &d->k, 2 * rows * H)) ||
        (rc = alloc((void **) &d->vt, 2 * (size_t) B * H * d->ldv)) ||
        (rc = alloc((void **) &d->o, 2 * rows * H)) ||
        (rc = alloc((void **) &d->h, 2 * rows * F)) ||
        (rc = alloc((void **) &d->jobs_dev, sizeof(GemvJob) * (nstreams + 3))) ||
        (rc = alloc((void **) &d->freq, sizeof(float) * (H / 2))) ||
        (rc = alloc((void **) &d->rope_cs, sizeof(float) * T * c.head_dim))) {
        tsk_dit_destroy(d);
        return rc;
    }
    d->q8 = c.weight_type == TSK_TYPE_Q8_0;
    if (d->q8 &&
        ((rc = alloc((void **) &d->qkv32, sizeof(float) * rows * 3 * H)) ||
         (rc = alloc((void **) &d->o32, sizeof(float) * rows * H)) ||
         (rc = alloc((void **) &d->qh, (size_t) rows * F)) ||
         (rc = alloc((void **) &d->dh, sizeof(float) * rows * (F / 32))) ||
         (rc = alloc((void **) &d->qx, (size_t) rows * F)) ||
         (rc = alloc((void **) &d->dx, sizeof(float) * rows * (F / 32))))) {
        tsk_dit_destroy(d);
        return rc;
    }
    {
        hipError_t se = hipStreamCreateWithFlags(&d->side, hipStreamNonBlocking);
        if (se == hipSuccess) se = hipEventCreateWithFlags(&d->ev_fork, hipEventDisableTiming);
        if (se == hipSuccess) se = hipEventCreateWithFlags(&d->ev_join, hipEventDisableTiming);
        if (se != hipSuccess) { tsk_dit_destroy(d); return hip_fail(se, "side stream"); }
    }
    // t-embedding frequencies exactly as the host code of mmdit.cpp:308-310
    std::vector<float> fr(H / 2);
    const float fscale_t = 10000.0f / c.t_max_period;
    for (int kk = 0; kk < H / 2; ++kk) fr[kk] = fscale_t * powf(10000.0f, -2.0f * (float) kk / (float) H);
    hipError_t e = hipMemcpy(d->freq, fr.data(), sizeof(float) * (H / 2), hipMemcpyHostToDevice);
    if (e != hipSuccess) { tsk_dit_destroy(d); return hip_fail(e, "hipMemcpy freq"); }
    // latent positions 0 .. max_latent - 1, freq_scale 1 (mmdit.cpp:96-99, :316-318)
    e = launch_rope_table(d->rope_cs, T, c.head_dim, powf(c.rope_theta, -2.0f / (float) c.head_dim), 1.0f, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) { tsk_dit_destroy(d); return hip_fail(e, "rope table"); }
    e = hipMemset(d->blob, 0, d->blob_bytes);
    if (e != hipSuccess) { tsk_dit_destroy(d); return hip_fail(e, "hipMemset"); }
    // V^T key positions past a call's token count are read (and multiplied by
    // P = 0) by the attention kernel: they must hold finite values
    e = hipMemset(d->vt, 0, 2 * (size_t) B * H * d->ldv);
    if (e != hipSuccess) { tsk_dit_destroy(d); return hip_fail(e, "hipMemset"); }

    // per-stream weights and adaLN job table
    std::vector<GemvJob> jobs;
    float *mp = d->mods;
    size_t soff = 0;
    auto mk = [&](StreamW s) {
        s.mod = mp;
        mp += (size_t) B * 6 * H;
        s.sched_off = soff;
        d->jobs_sched_off.push_back(soff);
        soff += (size_t) 6 * H;
        GemvJob j;
        j.w = s.ada_w; j.bias = s.ada_b; j.x = d->cvec; j.out = s.mod; j.M = s.nmod * H;
        j.silu_out = 0; j.ld_out = (int64_t) s.nmod * H;
        jobs.push_back(j);
        return s;
    };
    for (int i = 0; i < nj; ++i) {
        d->joint_lat.push_back(mk(stream_weights(d, "joint_blocks." + std::to_string(i) + ".latent_block", false)));
        d->joint_txt.push_back(mk(stream_weights(d, "joint_blocks." + std::to_string(i) + ".text_block", i == nj - 1)));
    }
    for (int i = 0; i < c.fused_depth; ++i) d->fused.push_back(mk(stream_weights(d, "fused_blocks." + std::to_string(i), false)));
    GemvJob fj;
    fj.w = wptr<uint16_t>(d, "final_layer.adaLN_modulation.1.weight");
    fj.bias = wptr<float>(d, "final_layer.adaLN_modulation.1.bias");
    fj.x = d->cvec;
    fj.out = mp;
    d->final_mod = mp;
    d->sched_final = soff;
    d->sched_row = soff + (size_t) 2 * H;
    d->jobs_sched_off.push_back(soff);
    fj.M = 2 * H;
    fj.silu_out = 0;
    fj.ld_out = 2 * H;
    jobs.push_back(fj);
    d->njobs = (int) jobs.size();
    // t_embed MLP (f32 activations): silu(W0 temb + b0) -> silu(W2 . + b2) = silu(cond)
    GemvJob t0, t2;
    t0.w = wptr<uint16_t>(d, "t_embed.mlp.0.weight"); t0.bias = wptr<float>(d, "t_embed.mlp.0.bias");
    t0.x = d->temb; t0.out = d->tmp_c; t0.M = H; t0.silu_out = 1; t0.ld_out = H;
    t2.w = wptr<uint16_t>(d, "t_embed.mlp.2.weight"); t2.bias = wptr<float>(d, "t_embed.mlp.2.bias");
    t2.x = d->tmp_c; t2.out = d->cvec; t2.M = H; t2.silu_out = 1; t2.ld_out = H;
    jobs.push_back(t0);
    jobs.push_back(t2);
    d->max_job_m = 6 * H;
    d->jobs_host = jobs;
    e = hipMemcpy(d->jobs_dev, jobs.data(), sizeof(GemvJob) * jobs.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) { tsk_dit_destroy(d); return hip_fail(e, "hipMemcpy jobs"); }
    *out = d;
    return TSK_OK;
}

extern "C" int tsk_dit_n_tensors(const tsk_dit *d) { return d ? (int) d->w.size() : 0; }

extern "C" int tsk_dit_tensor_info(const tsk_dit *d, int i, const char **name, int64_t ne[4]) {
    if (!d || i < 0 || i >= (int) d->w.size()) return fail(TSK_ERR_INVALID_ARG, "tensor index %d", i);
    if (name) *name = d->w[i].name.c_str();
    if (ne) { ne[0] = d->w[i].ne0; ne[1] = d->w[i].ne1; ne[2] = 1; ne[3] = 1; }
    return TSK_OK;
}

namespace {

// fp32 -> fp16 bits, round to nearest even (the GGML_FP32_TO_FP16 of a
// Q8_0 block scale)
uint16_t host_f16_bits(float f) {
    const _Float16 h = (_Float16) f;
    uint16_t b;
    memcpy(&b, &h, 2);
    return b;
}

// Q8_0 blocks [M][K / 32] of 34 bytes -> the driver's planes (int8 [M][K],
// fp16 d [M][K / 32]) on the device; rows already in the driver's order
int upload_q8_blocks(tsk_dit *d, const WInfo &wi, const uint8_t *blocks) {
    const int64_t K = wi.ne0, M = wi.ne1, KB = K / 32;
    std::vector<uint8_t> planes(tsk_q8_0_split_nbytes(K, M));
    uint16_t *dp = (uint16_t *) (planes.data() + (size_t) (M * K));
    for (int64_t m = 0; m < M; ++m)
        for (int64_t kb = 0; kb < KB; ++kb) {
            const uint8_t *blk = blocks + (m * KB + kb) * 34;
            memcpy(&dp[m * KB + kb], blk, 2);
            memcpy(&planes[(size_t) (m * K + kb * 32)], blk + 2, 32);
        }
    return hipcheck(hipMemcpy(d->blob + wi.offset, planes.data(), planes.size(), hipMemcpyHostToDevice), "set_tensor copy");
}

// rows of the (h d j)-interleaved QKV output order -> [q | k | v] blocks:
// source row 3 i + j -> destination row j H + i (rows of rowbytes bytes)
std::vector<uint8_t> permute_qkv_rows(const void *src, int H, size_t rowbytes) {
    std::vector<uint8_t> out((size_t) 3 * H * rowbytes);
    for (int64_t i = 0; i < H; ++i)
        for (int j = 0; j < 3; ++j)
            memcpy(&out[(size_t) (j * H + i) * rowbytes], (const uint8_t *) src + (size_t) (3 * i + j) * rowbytes, rowbytes);
    return out;
}

}  // namespace

extern "C" int tsk_dit_tensor_type(const tsk_dit *d, int i) {
    if (!d || i < 0 || i >= (int) d->w.size()) return fail(TSK_ERR_INVALID_ARG, "tensor index %d", i);
    const WInfo &wi = d->w[i];
    return wi.q8 ? TSK_TYPE_Q8_0 : wi.matrix ? TSK_TYPE_BF16 : TSK_TYPE_F32;
}

extern "C" int tsk_dit_set_tensor_q8_0(tsk_dit *d, const char *name, const void *blocks, size_t nbytes) {
    if (!d || !name || !blocks) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = d->idx.find(name);
    if (it == d->idx.end()) return fail(TSK_ERR_INVALID_ARG, "unknown tensor '%s'", name);
    const WInfo &wi = d->w[it->second];
    if (!wi.q8) return fail(TSK_ERR_TYPE, "'%s' is not stored as Q8_0 by this driver", name);
    const size_t rowbytes = (size_t) (wi.ne0 / 32) * 34;
    if (nbytes != rowbytes * (size_t) wi.ne1)
        return fail(TSK_ERR_SHAPE, "'%s' has %zu bytes of Q8_0 blocks, got %zu", name, rowbytes * (size_t) wi.ne1, nbytes);
    if (wi.qkv_perm) {
        const std::vector<uint8_t> pb = permute_qkv_rows(blocks, d->cfg.hidden, rowbytes);
        return upload_q8_blocks(d, wi, pb.data());
    }
    return upload_q8_blocks(d, wi, (const uint8_t *) blocks);
}

// host f32 -> device (bf16 for matrices, Q8_0 for the Q8_0 driver's block
// projections), with the (h d j) -> [q|k|v] row permutation
extern "C" int tsk_dit_set_tensor(tsk_dit *d, const char *name, const float *src, int64_t n) {
    if (!d || !name || !src) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = d->idx.find(name);
    if (it == d->idx.end()) return fail(TSK_ERR_INVALID_ARG, "unknown tensor '%s'", name);
    const WInfo &wi = d->w[it->second];
    if (n != wi.ne0 * wi.ne1) return fail(TSK_ERR_SHAPE, "'%s' has %lld elements, got %lld", name, (long long) (wi.ne0 * wi.ne1), (long long) n);
    const int H = d->cfg.hidden;
    std::vector<float> perm;
    const float *s = src;
    if (wi.qkv_perm) {
        // source row r = 3*i + j (i = h*64 + d) -> destination row j*H + i
        const int64_t rowlen = wi.matrix ? wi.ne0 : 1;
        perm.resize((size_t) n);
        for (int64_t i = 0; i < H; ++i)
            for (int j = 0; j < 3; ++j)
                memcpy(&perm[(size_t) ((j * H + i) * rowlen)], src + (3 * i + j) * rowlen, sizeof(float) * rowlen);
        s = perm.data();
    }
    char *dst = d->blob + wi.offset;
    if (wi.q8) {
        // ggml's reference Q8_0 quantizer (quantize_row_q8_0_ref; the gguf-py
        // converter's quantize, convert/quantize_gguf.py:41, is bit-identical):
        // d = amax / 127, q = round-half-away(x / d), d stored as fp16
        const int64_t K = wi.ne0, M = wi.ne1, KB = K / 32;
        std::vector<uint8_t> blocks((size_t) (M * KB) * 34);
        for (int64_t bi = 0; bi < M * KB; ++bi) {
            const float *x = s + bi * 32;
            float amax = 0.0f;
            for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
            const float dd = amax / 127.0f;
            const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
            uint8_t *blk = &blocks[(size_t) bi * 34];
            const uint16_t h = host_f16_bits(dd);
            memcpy(blk, &h, 2);
            for (int j = 0; j < 32; ++j) blk[2 + j] = (uint8_t) (int8_t) roundf(x[j] * id);
        }
        return upload_q8_blocks(d, wi, blocks.data());
    }
    if (!wi.matrix) {
        float a = 0.0f;
        for (int64_t i = 0; i < n; ++i) a = fmaxf(a, fabsf(src[i]));
        d->w[it->second].amax = a;
    }
    hipError_t e;
    if (wi.matrix) {
        std::vector<uint16_t> bf((size_t) n);
        for (int64_t i = 0; i < n; ++i) {
            uint32_t x;
            memcpy(&x, &s[i], 4);
            if ((x & 0x7fffffffu) > 0x7f800000u) bf[i] = (uint16_t) ((x >> 16) | 64u);
            else bf[i] = (uint16_t) ((x + (0x7fffu + ((x >> 16) & 1u))) >> 16);
        }
        if (wi.tiled) {
            // rows of K = ne0 -> 16 x 32 MFMA tiles (tiled_index), 8 elements at a time
            const int64_t K = wi.ne0, M = wi.ne1;
            std::vector<uint16_t> t((size_t) n);
            for (int64_t m = 0; m < M; ++m)
                for (int64_t k = 0; k < K; k += 8)
                    memcpy(&t[(size_t) tiled_index(m, k, K)], &bf[(size_t) (m * K + k)], 16);
            bf.swap(t);
        }
        e = hipMemcpy(dst, bf.data(), 2 * (size_t) n, hipMemcpyHostToDevice);
    } else {
        e = hipMemcpy(dst, s, 4 * (size_t) n, hipMemcpyHostToDevice);
    }
    return hipcheck(e, "set_tensor copy");
}

// ------------------------------------------------------------------ forward
namespace {

// One stream (latent or text) of a block as seen by the grouped launches.
struct StreamRun {
    const StreamW *w;
    float *x;               // f32 residual rows [B * S][H]
    int S;                  // tokens per batch row
    int tok_off;            // offset of this stream in the joint token order
    int rope;               // RoPE on q/k (latent stream)
    uint16_t *xn, *h;       // bf16 LN outputs / GELU outputs of this stream
    float *part;            // split-K partials of this stream
    int64_t row_off;        // first row of this stream in the capacity layout (xn, h, qx, ...)
    // residual update still owed from the previous projection (split-K partials)
    const float *pend_bias = nullptr, *pend_gate = nullptr;
    int64_t pend_ld_gate = 0;   // row stride of the owing block's modulation
    int pend_split = 0;
};

// adaLN outputs of a block for the running call: its own [B][nmod * H] rows,
// or one schedule row shared by the batch (row stride 0)
const float *mod_of(const tsk_dit *d, const StreamW &w) { return d->cur_sched ? d->cur_sched + w.sched_off : w.mod; }
int64_t mod_ld(const tsk_dit *d, const StreamW &w) { return d->cur_sched ? 0 : (int64_t) w.nmod * d->cfg.hidden; }

LnStream ln_stream(const StreamRun &r, int B, int H, int64_t ldm, const float *shift, const float *scale, void *y) {
    LnStream l;
    memset(&l, 0, sizeof(l));
    l.x = r.x; l.ld_x = H;
    if (r.pend_split) {
        l.part = r.part; l.nsplit = r.pend_split; l.part_stride = (int64_t) B * r.S * H;
        l.bias = r.pend_bias; l.gate = r.pend_gate; l.ld_gate = r.pend_ld_gate;
    }
    l.shift = shift; l.scale = scale; l.ld_mod = ldm;
    l.y = y; l.ld_y = H;
    l.rows = B * r.S; l.rows_per_b = r.S;
    return l;
}

GemmProblem gemm_problem(const void *x, int64_t ld_x, const uint16_t *w, const float *bias, void *y, int64_t ld_y,
                         int N, int K, int M) {
    GemmProblem q;
    memset(&q, 0, sizeof(q));
    q.x = x; q.w = w; q.w_tiled = 1; q.bias = bias; q.y = y;
    q.ld_x = ld_x; q.ld_w = K; q.ld_y = ld_y;
    q.M = M; q.N = N; q.K = K; q.splits = 1;
    return q;
}

int gemm_cfg_for(const tsk_dit *d, int role, int rows);

// split-K slices of the BF16 driver's linear1 (K = 1024) by latent tokens per
// batch item (never by batch, so that batch rows stay independent bit for
// bit): two below 550, where 16 x 64-row tiles per few hundred rows leave
// most CUs idle, one from there (MI355X, 30 s: the GEMM 9.4 -> 9.1 us and its
// LN reading one slice instead of two, 422 -> 426 steps/s; at 9 s one slice
// loses 670 -> 654)
int ksplit_out_for(const tsk_dit *d, int seq) {
    if (!d->ksplit_auto) return d->ksplit_out;
    return seq >= 550 ? 1 : 2;
}

// LN + modulate of every stream (paying the residual updates they owe) into
// xn (bf16), or into the Q8_0 planes qx / dx for the Q8_0 driver
int run_ln(tsk_dit *d, StreamRun *r, int ns, int B, int which, hipStream_t st) {
    const tsk_dit_config &c = d->cfg;
    const int H = c.hidden;
    LnGroup g;
    memset(&g, 0, sizeof(g));
    g.nstream = ns; g.H = H; g.eps = c.ln_eps; g.y_mode = d->q8 ? LN_Y_Q8 : LN_Y_BF16;
    double rows = 0.0, pbytes = 0.0;
    for (int i = 0; i < ns; ++i) {
        const StreamW &w = *r[i].w;
        const int64_t ldm = mod_ld(d, w);
        // which = 0: shift_msa / scale_msa (mod 0, 1); 1: shift_mlp / scale_mlp (mod 3, 4)
        const float *m = mod_of(d, w);
        const float *sh = m + (which ? 3 : 0) * H, *sc = m + (which ? 4 : 1) * H;
        g.s[i] = ln_stream(r[i], B, H, ldm, sh, sc, r[i].xn);
        if (d->q8) {
            g.s[i].y = d->qx + r[i].row_off * H;
            g.s[i].yd = d->dx + r[i].row_off * (H / 32);
        }
        rows += (double) B * r[i].S;
        pbytes += 4.0 * r[i].pend_split * B * r[i].S * H;
        r[i].pend_split = 0;
    }
    // BF16 driver: the LN workgroups fetch the weights of the projections that
    // follow into the L2 of the XCDs that will read them (qkv and linear1
    // after the attention LN, fc1 and fc2 after the MLP LN). The LN then ends
    // only when those loads have landed; measured on MI355X this pays from
    // ~800 latent rows (T = 400: 1.94 -> 1.92 ms, 30 s: 2.44-2.46 -> 2.33-2.39
    // ms per step on different boxes) and breaks even at 388 (9 s), where the
    // LN kernels are too short to cover the extra 16-32 MB of weight reads:
    // on from 512 rows.
    const int rows0 = B * r[0].S;
    const int pf_mode = tuning().l2_prefetch;
    L2PrefetchList pf;
    memset(&pf, 0, sizeof(pf));
    if (!d->q8 && (pf_mode > 0 || (pf_mode < 0 && rows0 >= 512))) {
        auto add = [&](const uint16_t *w, int K, int M, int role, int splits) {
            const int bm = gemm_ks_bm(gemm_cfg_for(d, role, rows0));
            L2Prefetch &f = pf.pf[pf.npf];
            f.w = w; f.kt_n = K / 32; f.rb_tile = bm / 16; f.rb_n = M / 16;
            f.tiles_m = (M + bm - 1) / bm; f.splits = splits;
            if ((f.tiles_m * f.splits) % 8 == 0 && f.kt_n % splits == 0) ++pf.npf;
        };
        for (int i = 0; i < ns; ++i) {
            const StreamW &w = *r[i].w;
            if (which == 0) add(w.qkv_w, H, 3 * H, 0, 1);
            else if (!w.pre_only) add(w.fc1_w, H, c.mlp_hidden, 2, 1);
        }
        for (int i = 0; i < ns; ++i) {
            const StreamW &w = *r[i].w;
            if (w.pre_only) continue;
            if (which == 0) add(w.l1_w, H, H, 1, ksplit_out_for(d, r[0].S));
            else add(w.fc2_w, c.mlp_hidden, H, 3, d->ksplit_fc2);
        }
    }
    Timed tm(d, TSK_ROLE_OTHER, 10.0 * rows * H, 14.0 * rows * H + pbytes, st);
    return hipcheck(launch_ln_group(g, st, pf.npf ? &pf : nullptr), "ln_group");
}

// Block GEMM tile shape by projection and activation rows of the larger
// stream, measured on MI355X over 194 .. 646 latent tokens (B = 2): below
// 550 rows 64 x 64 cooperative tiles of 64-wide stages (cfg 30); up to 1100
// rows the same for qkv, 64 x 64 tiles of 32-wide stages for out (cfg 22)
// and 128 x 64 tiles of 64-wide stages for the MLP (cfg 28); beyond, 128 x 64
// tiles of two 64-wide stages (cfg 29), 64 x 64 for out (cfg 30). The tile
// shape does not change any summation order.
int gemm_cfg_for(const tsk_dit *d, int role, int rows) {
    if (d->gemm_cfg[role]) return d->gemm_cfg[role];
    if (rows >= 1100) return role == 1 ? 30 : 29;
    if (rows < 550) return 30;
    static const int mid[4] = {30, 22, 28, 28};   // qkv, out, fc1, fc2
    return mid[role];
}

int run_qkv(tsk_dit *d, StreamRun *r, int ns, int B, int Ntot, hipStream_t st) {
    const tsk_dit_config &c = d->cfg;
    const int H = c.hidden;
    GemmGroup g;
    memset(&g, 0, sizeof(g));
    g.nprob = ns;
    double fl = 0.0, by = 0.0;
    for (int i = 0; i < ns; ++i) {
        const int rows = B * r[i].S;
        GemmProblem &q = g.p[i];
        q = gemm_problem(r[i].xn, H, r[i].w->qkv_w, r[i].w->qkv_b, nullptr, 0, rows, H, 3 * H);
        q.qn_w = r[i].w->qn; q.kn_w = r[i].w->kn;
        q.q = d->q; q.k = d->k; q.vt = d->vt; q.ldv = d->ldv;
        q.v_rows = tuning().attn_vrows != 0;   // V as rows like k (read by the attention's transposing LDS reads)
        q.seq = r[i].S; q.Ntot = Ntot; q.tok_off = r[i].tok_off; q.rope = r[i].rope;
        q.theta_scale = powf(c.rope_theta, -2.0f / (float) c.head_dim);
        q.freq_scale = 1.0f;
        q.eps = c.qk_eps;
        q.q_scale = 1.4426950408889634f / sqrtf((float) c.head_dim);   // scale * log2(e), see attention()
        q.rope_cs = r[i].rope ? d->rope_cs : nullptr;
        fl += 2.0 * rows * H * 3.0 * H;
        by += 2.0 * 3 * H * H + 2.0 * rows * H + 2.0 * rows * 3 * H + 12.0 * H;
    }
    Timed tm(d, TSK_ROLE_QKV, fl, by, st);
    return hipcheck(launch_gemm_ks(g, EPI_QKV, gemm_cfg_for(d, 0, B * r[0].S), st), "qkv gemm");
}

// linear1 on the attention output (o rows of each stream: o[b][tok_off + s]),
// split-K partials; the residual update is paid by the next run_ln
int run_out(tsk_dit *d, StreamRun *r, int ns, int B, int Ntot, hipStream_t st) {
    const int H = d->cfg.hidden;
    GemmGroup g;
    memset(&g, 0, sizeof(g));
    double fl = 0.0, by = 0.0;
    for (int i = 0; i < ns; ++i) {
        if (r[i].w->pre_only) continue;
        const int rows = B * r[i].S;
        GemmProblem &q = g.p[g.nprob++];
        q = gemm_problem(d->o + (size_t) r[i].tok_off * H, H, r[i].w->l1_w, nullptr, r[i].part, H, rows, H, H);
        q.x_group_rows = r[i].S;
        q.x_group_stride = (int64_t) Ntot * H;
        q.splits = ksplit_out_for(d, r[0].S);
        r[i].pend_split = q.splits;
        r[i].pend_bias = r[i].w->l1_b;
        r[i].pend_gate = mod_of(d, *r[i].w) + 2 * H;   // gate_msa
        r[i].pend_ld_gate = mod_ld(d, *r[i].w);
        fl += 2.0 * rows * H * H;
        by += 2.0 * H * H + 2.0 * rows * H + 4.0 * q.splits * rows * H;
    }
    if (!g.nprob) return TSK_OK;
    Timed tm(d, TSK_ROLE_OUT, fl, by, st);
    return hipcheck(launch_gemm_ks(g, EPI_PARTIAL, gemm_cfg_for(d, 1, B * r[0].S), st), "linear1 gemm");
}

int run_mlp(tsk_dit *d, StreamRun *r, int ns, int B, hipStream_t st) {
    const int H = d->cfg.hidden, F = d->cfg.mlp_hidden;
    GemmGroup g1, g2;
    memset(&g1, 0, sizeof(g1));
    memset(&g2, 0, sizeof(g2));
    double fl = 0.0, by1 = 0.0, by2 = 0.0;
    for (int i = 0; i < ns; ++i) {
        if (r[i].w->pre_only) continue;
        const int rows = B * r[i].S;
        g1.p[g1.nprob++] = gemm_problem(r[i].xn, H, r[i].w->fc1_w, r[i].w->fc1_b, r[i].h, F, rows, H, F);
        GemmProblem &q = g2.p[g2.nprob++];
        q = gemm_problem(r[i].h, F, r[i].w->fc2_w, nullptr, r[i].part, H, rows, F, H);
        q.splits = d->ksplit_fc2;
        r[i].pend_split = d->ksplit_fc2;
        r[i].pend_bias = r[i].w->fc2_b;
        r[i].pend_gate = mod_of(d, *r[i].w) + 5 * H;   // gate_mlp
        r[i].pend_ld_gate = mod_ld(d, *r[i].w);
        fl += 2.0 * rows * H * F;
        by1 += 2.0 * F * H + 2.0 * rows * H + 2.0 * rows * F;
        by2 += 2.0 * H * F + 2.0 * rows * F + 4.0 * d->ksplit_fc2 * rows * H;
    }
    if (!g1.nprob) return TSK_OK;
    int rc;
    {
        Timed tm(d, TSK_ROLE_FC1, fl, by1, st);
        rc = hipcheck(launch_gemm_ks(g1, EPI_GELU_BF16, gemm_cfg_for(d, 2, B * r[0].S), st), "fc1 gemm");
    }
    if (rc) return rc;
    Timed tm(d, TSK_ROLE_FC2, fl, by2, st);
    return hipcheck(launch_gemm_ks(g2, EPI_PARTIAL, gemm_cfg_for(d, 3, B * r[0].S), st), "fc2 gemm");
}

// ---- the Q8_0 driver's block projections (weight_type Q8_0): every
// projection reads Q8_0 planes of f32 activations (ggml_mul_mat's conversion
// of src1 for a Q8_0 weight) and runs gemm_q8c: exact int32 block sums, fp32
// rescale and accumulation

GemmParams q8_problem(const tsk_dit *d, const Q8W &w, const StreamRun &r, int B, int K, int M, const float *bias) {
    GemmParams p;
    memset(&p, 0, sizeof(p));
    p.qw = w.q; p.dw = w.d;
    p.qx = d->qx + r.row_off * K;
    p.dx = d->dx + r.row_off * (K / 32);
    p.M = M; p.N = B * r.S; p.K = K;
    p.bias = bias;
    p.rows_per_gate = 1;
    return p;
}

double q8_bytes(int N, int K, int M, double out_bytes) {
    return (double) M * K * (1.0 + 2.0 / 32) + (double) N * K * (1.0 + 4.0 / 32) + (double) N * M * out_bytes;
}

// the Q8_0 projections of the active streams: a joint block's two in one
// launch (launch_gemm_q8_pair), one stream alone otherwise
int q8_launch(tsk_dit *d, const GemmParams *ps, int n, int role, double fl, double by, const char *what,
              hipStream_t st) {
    if (n < 1) return TSK_OK;
    Timed tm(d, role, fl, by, st);
    return hipcheck(n == 2 ? launch_gemm_q8_pair(ps[0], ps[1], st) : launch_gemm_q8(ps[0], st), what);
}

// QKV GEMM with the RMSNorm / RoPE / fp16 scatter into the attention
// operands as its epilogue (or, with Tuning::q8_qkv_fused off, into f32 rows
// and then the scatter kernel: the same bits)
int run_qkv_q8(tsk_dit *d, StreamRun *r, int ns, int B, int Ntot, hipStream_t st) {
    const tsk_dit_config &c = d->cfg;
    const int H = c.hidden;
    const bool fused = tuning().q8_qkv_fused != 0;
    int rc;
    QkvScatter qs[2];
    double rows = 0.0;
    for (int i = 0; i < ns; ++i) {
        QkvScatter &q = qs[i];
        memset(&q, 0, sizeof(q));
        q.qkv = d->qkv32 + r[i].row_off * 3 * H;
        q.ld = 3 * H;
        q.qn_w = r[i].w->qn; q.kn_w = r[i].w->kn;
        q.rope_cs = r[i].rope ? d->rope_cs : nullptr;
        q.q = d->q; q.k = d->k; q.vt = d->vt; q.ldv = d->ldv;
        q.seq = r[i].S; q.Ntot = Ntot; q.tok_off = r[i].tok_off; q.rope = r[i].rope;
        q.nh = c.n_head; q.rows = B * r[i].S;
        q.eps = c.qk_eps;
        q.q_scale = 1.4426950408889634f / sqrtf((float) c.head_dim);   // scale * log2(e), as run_qkv
        q.v_rows = tuning().attn_vrows != 0;
        rows += (double) B * r[i].S;
    }
    {
        GemmParams ps[2];
        double fl = 0.0, by = 0.0;
        for (int i = 0; i < ns; ++i) {
            GemmParams &p = ps[i];
            p = q8_problem(d, r[i].w->qkv_q, r[i], B, H, 3 * H, r[i].w->qkv_b);
            if (fused) {
                p.epi = EPI_QKV_ATTN;
                p.qs = qs[i];
            } else {
                p.y = d->qkv32 + r[i].row_off * 3 * H;
                p.ld_y = 3 * H;
                p.epi = EPI_STORE;
            }
            fl += 2.0 * p.N * H * 3.0 * H;
            by += q8_bytes(p.N, H, 3 * H, fused ? 2 : 4);
        }
        if ((rc = q8_launch(d, ps, ns, TSK_ROLE_QKV, fl, by, "qkv q8 gemm", st))) return rc;
    }
    if (fused) return TSK_OK;
    // both streams of a joint block in one launch
    Timed tm(d, TSK_ROLE_OTHER, 10.0 * rows * 3 * H, 12.0 * rows * 3 * H, st);
    return hipcheck(ns == 2 ? launch_qkv_scatter2(qs[0], qs[1], st) : launch_qkv_scatter(qs[0], st), "qkv scatter");
}

// split-K partials of a Q8_0 projection into the stream's partial slices;
// the next LN adds gate * (sum of the slices + bias) to the residual, as for
// the BF16 projections
void q8_partials(const tsk_dit *d, GemmParams &p, StreamRun &r, int B, int splits, const float *bias, int gate_chunk) {
    const int H = d->cfg.hidden;
    p.bias = nullptr;
    p.epi = EPI_STORE;
    p.y = r.part; p.ld_y = H;
    p.splits = splits;
    p.part_stride = (int64_t) B * r.S * H;
    r.pend_split = splits;
    r.pend_bias = bias;
    r.pend_gate = mod_of(d, *r.w) + gate_chunk * H;
    r.pend_ld_gate = mod_ld(d, *r.w);
}

// linear1 on the attention output of each stream as Q8_0 planes (the
// attention kernel's own Q8_0 output, or its f32 output quantized per
// stream), split-K partials; gate_msa * (linear1 + bias) is added to the
// residual by the next LN
int run_out_q8(tsk_dit *d, StreamRun *r, int ns, int B, int Ntot, hipStream_t st) {
    const int H = d->cfg.hidden;
    int rc;
    {
        // the attention output of every stream that has a linear1, as Q8_0 planes
        // (one launch for a joint block's two streams)
        QuantRows qr[2];
        int nq = 0;
        double rows = 0.0;
        for (int i = 0; i < ns; ++i) {
            if (r[i].w->pre_only) continue;
            QuantRows &q = qr[nq++];
            q.x = d->o32 + (size_t) r[i].tok_off * H; q.ld_x = H;
            q.N = B * r[i].S; q.K = H;
            q.qx = d->qx + r[i].row_off * H; q.dx = d->dx + r[i].row_off * (H / 32);
            q.grp = r[i].S; q.gstride = Ntot;
            rows += (double) q.N;
        }
        if (nq && !tuning().attn_q8) {
            Timed tm(d, TSK_ROLE_OTHER, 3.0 * rows * H, 5.125 * rows * H, st);
            rc = hipcheck(nq == 2 ? launch_quantize_rows_q8_pair(qr[0], qr[1], st)
                                  : launch_quantize_rows_q8(qr[0].x, 1, qr[0].ld_x, qr[0].N, qr[0].K, qr[0].qx, qr[0].dx,
                                                            st, qr[0].grp, qr[0].gstride),
                          "linear1 quantize");
            if (rc) return rc;
        }
    }
    GemmParams ps[2];
    int n = 0;
    double fl = 0.0, by = 0.0;
    for (int i = 0; i < ns; ++i) {
        if (r[i].w->pre_only) continue;
        GemmParams &p = ps[n++];
        p = q8_problem(d, r[i].w->l1_q, r[i], B, H, H, nullptr);
        q8_partials(d, p, r[i], B, d->ksplit_out, r[i].w->l1_b, 2);   // gate_msa
        fl += 2.0 * p.N * H * H;
        by += q8_bytes(p.N, H, H, 4 * p.splits);
    }
    return q8_launch(d, ps, n, TSK_ROLE_OUT, fl, by, "linear1 q8 gemm", st);
}

// fc1 of every stream with GELU and the Q8_0 conversion of its output in the
// epilogue (into qh / dh: fc1 still reads qx), then fc2 as split-K partials
// (gate_mlp * (fc2 + bias) is added to the residual by the next LN)
int run_mlp_q8(tsk_dit *d, StreamRun *r, int ns, int B, hipStream_t st) {
    const int H = d->cfg.hidden, F = d->cfg.mlp_hidden;
    int rc;
    GemmParams p1[2], p2[2];
    int n = 0;
    double fl = 0.0, by1 = 0.0, by2 = 0.0;
    for (int i = 0; i < ns; ++i) {
        if (r[i].w->pre_only) continue;
        GemmParams &p = p1[n];
        p = q8_problem(d, r[i].w->fc1_q, r[i], B, H, F, r[i].w->fc1_b);
        p.y = d->qh + r[i].row_off * F;
        p.ld_y = F;
        p.yd = d->dh + r[i].row_off * (F / 32);
        p.epi = EPI_GELU_Q8;
        GemmParams &q = p2[n++];
        q = q8_problem(d, r[i].w->fc2_q, r[i], B, F, H, nullptr);
        q.qx = d->qh + r[i].row_off * F;
        q.dx = d->dh + r[i].row_off * (F / 32);
        q8_partials(d, q, r[i], B, d->ksplit_fc2, r[i].w->fc2_b, 5);   // gate_mlp
        fl += 2.0 * p.N * H * F;
        by1 += q8_bytes(p.N, H, F, 1.125);
        by2 += q8_bytes(q.N, F, H, 4 * q.splits);
    }
    if ((rc = q8_launch(d, p1, n, TSK_ROLE_FC1, fl, by1, "fc1 q8 gemm", st))) return rc;
    return q8_launch(d, p2, n, TSK_ROLE_FC2, fl, by2, "fc2 q8 gemm", st);
}

int attention(tsk_dit *d, const StreamRun *r, int ns, int B, int Ntot, hipStream_t st);

// one block of the Q8_0 driver over the streams r[0..ns)
int block_q8(tsk_dit *d, StreamRun *r, int ns, int B, int Ntot, hipStream_t st) {
    int rc;
    if ((rc = run_ln(d, r, ns, B, 0, st))) return rc;
    if ((rc = run_qkv_q8(d, r, ns, B, Ntot, st))) return rc;
    if ((rc = attention(d, r, ns, B, Ntot, st))) return rc;
    if ((rc = run_out_q8(d, r, ns, B, Ntot, st))) return rc;
    const int nmlp = ns == 2 && r[1].w->pre_only ? 1 : ns;
    if ((rc = run_ln(d, r, nmlp, B, 1, st))) return rc;
    return run_mlp_q8(d, r, nmlp, B, st);
}

// Attention over the concatenated q/k/vt of the streams in r[0..ns). q was
// written pre-multiplied by scale * log2(e) (run_qkv). q and k are RMS-normed
// (|x / rms(x)| = 8 for 64 dims) times w, and RoPE is a rotation, so every
// logit obeys |q.k| * scale * log2(e) <= 64 * scale * log2(e) * max|w_q| *
// max|w_k| over the streams: under ATTN_LOGIT_BOUND the kernel needs no
// running max.
int attention(tsk_dit *d, const StreamRun *r, int ns, int B, int Ntot, hipStream_t st) {
    const tsk_dit_config &c = d->cfg;
    AttnFastParams p;
    memset(&p, 0, sizeof(p));
    // Q8_0 driver: f32 output, which linear1 quantizes to Q8_0 (the flash
    // attention node's F32 result, src/mmdit.cpp:91-93)
    const int es = d->q8 ? 4 : 2;
    p.q = d->q; p.k = d->k; p.vt = d->vt; p.o = d->q8 ? (void *) d->o32 : (void *) d->o;
    p.q_type = TSK_TYPE_F16; p.k_bf16 = 0; p.out_bf16 = d->q8 ? 0 : 1;
    p.Nq = p.Nkv = Ntot; p.H = c.n_head; p.B = B;
    p.q_nb1 = p.k_nb1 = 128;
    p.q_nb2 = p.k_nb2 = (int64_t) 128 * Ntot;
    p.q_nb3 = p.k_nb3 = (int64_t) 128 * Ntot * c.n_head;
    p.vt_bh = (int64_t) 64 * d->ldv;
    p.ldv = d->ldv;
    p.o_nb1 = 64 * es; p.o_nb2 = (int64_t) es * c.hidden; p.o_nb3 = (int64_t) es * c.hidden * Ntot;
    p.c = 1.4426950408889634f / sqrtf((float) c.head_dim);
    p.q_prescaled = 1;
    float aq = 0.0f, ak = 0.0f;
    for (int i = 0; i < ns; ++i) {
        aq = fmaxf(aq, d->w[r[i].w->qn_idx].amax);
        ak = fmaxf(ak, d->w[r[i].w->kn_idx].amax);
    }
    // 1 % margin for the fp16 rounding of q and k
    p.bounded = 1.01f * (float) c.head_dim * p.c * aq * ak <= ATTN_LOGIT_BOUND;
    p.force_cfg = d->attn_cfg;
    p.rule_b = d->cfg.max_batch;
    if (tuning().attn_vrows) {
        // the QKV epilogue (BF16 or Q8_0) wrote V as fp16 rows [B][n_head][Ntot][64] into vt
        p.v_rows = 1;
        p.v = d->vt;
        p.v_nb1 = 128; p.v_nb2 = (int64_t) 128 * Ntot; p.v_nb3 = (int64_t) 128 * Ntot * c.n_head;
    }
    if (!d->q8 && tuning().attn_xcd) {
        // the BF16 QKV GEMM's XCD split (weight tiles of bm rows, tile m on
        // XCD m % 8) puts head h's q / k / V^T in the L2 of XCD (h / (bm / 64)) % 8
        const int bm = gemm_ks_bm(gemm_cfg_for(d, 0, B * r[0].S));
        if (bm % 64 == 0 && (3 * c.hidden / bm) % 8 == 0) p.xcd_hdiv = bm / 64;
    }
    if (d->q8 && tuning().attn_q8) {
        // linear1's Q8_0 activations straight from the attention (the streams
        // that have a linear1), as quantize_rows_q8 would make them from o32
        for (int i = 0; i < ns; ++i) {
            if (r[i].w->pre_only) continue;
            p.q8_tok[p.q8_ns] = r[i].tok_off;
            p.q8_S[p.q8_ns] = r[i].S;
            p.q8_row[p.q8_ns] = (int) r[i].row_off;
            ++p.q8_ns;
        }
        if (p.q8_ns) {
            p.q8x = d->qx;
            p.q8d = d->dx;
        }
    }
    const double nn = (double) Ntot * Ntot;
    Timed tm(d, TSK_ROLE_ATTN, 4.0 * B * c.n_head * nn * c.head_dim, 4.0 * 2.0 * B * Ntot * c.hidden, st);
    return hipcheck(launch_attn_fast(p, st), "attention");
}

// The adaLN conditioning of one forward call: timestep embedding, t_embed MLP
// and every block's modulations for the call's B rows of t. The jobs of the
// first jmain streams run on the caller's stream, the rest on the side stream
// (the caller's stream waits on d->ev_join before the first block that needs
// them).
int run_conditioning(tsk_dit *d, int B, const float *t_host, int jmain, hipStream_t st) {
    const tsk_dit_config &c = d->cfg;
    const int H = c.hidden, nj = c.depth - c.fused_depth;
    hipError_t e;
    // timestep frequency embedding [cos(t f), sin(t f)] (mmdit.cpp:305-314); t by value
    TimeVals tv;
    for (int b = 0; b < 32; ++b) tv.t[b] = b < B ? t_host[b] : 0.0f;
    e = launch_timestep_embed(d->freq, tv, B, H, d->temb, st);
    if (e != hipSuccess) return hip_fail(e, "timestep embed");
    // t_embed MLP -> silu(cond) (mmdit.cpp:158-160, :209), f32 activations
    {
        Timed tm(d, TSK_ROLE_ADALN, 4.0 * B * H * H, 4.0 * H * H, st);
        if ((e = launch_gemv_jobs(d->jobs_dev + d->njobs, 1, H, B, H, st)) != hipSuccess) return hip_fail(e, "t_embed.0");
        if ((e = launch_gemv_jobs(d->jobs_dev + d->njobs + 1, 1, H, B, H, st)) != hipSuccess) return hip_fail(e, "t_embed.2");
    }
    // every adaLN modulation of the step: the jobs of the first two joint blocks
    // on the caller's stream, all later ones (the bulk of the 352 MB of adaLN
    // weights at d = 1024, HBM-bound) on the side stream, where they overlap
    // the first blocks
    {
        const double per = 6.0 * H * H;   // weight elements of one 6H-output job
        Timed tm(d, TSK_ROLE_ADALN, 2.0 * B * per * jmain, 2.0 * per * jmain, st);
        if ((e = launch_gemv_jobs(d->jobs_dev, jmain, d->max_job_m, B, H, st)) != hipSuccess)
            return hip_fail(e, "adaln gemv");
    }
    if ((e = hipEventRecord(d->ev_fork, st)) != hipSuccess) return hip_fail(e, "fork");
    if ((e = hipStreamWaitEvent(d->side, d->ev_fork, 0)) != hipSuccess) return hip_fail(e, "fork");
    {
        const double mtot = (double) H * (6.0 * (2 * nj + c.fused_depth) - 4.0 + 2.0) - 6.0 * H * jmain;
        Timed tm(d, TSK_ROLE_ADALN, 2.0 * B * mtot * H, 2.0 * mtot * H, d->side);
        if ((e = launch_gemv_jobs(d->jobs_dev + jmain, d->njobs - jmain, d->max_job_m, B, H, d->side)) != hipSuccess)
            return hip_fail(e, "adaln gemv");
    }
    if ((e = hipEventRecord(d->ev_join, d->side)) != hipSuccess) return hip_fail(e, "join");
    return TSK_OK;
}

// latent_d: [B][T][latent_dim] (token-major, the sampler's own state) or,
// with latent_cm, [B][latent_dim][T] (ne0 = T, ts_dit::forward's input);
// flow_d: [B][T][latent_dim] (ne0 = latent_dim, ts_dit::forward's output)
int forward_impl(tsk_dit *d, int B, int T, const float *latent_d, bool latent_cm, const float *t_host,
                 const float *text_d, float *flow_d, hipStream_t st) {
    const tsk_dit_config &c = d->cfg;
    const int H = c.hidden, St = c.text_seq, nj = c.depth - c.fused_depth;
    hipError_t e;
    int rc;
    // a sampler step with a conditioning schedule reads its modulations from
    // the schedule row (d->cur_sched); otherwise they are computed here
    const int jmain = 2 * (nj < 2 ? nj : 2);
    // input projection (f32 activations, fp32 accumulation) and text stream
    // copy first: the conditioning's later adaLN GEMVs fill the chip from the
    // side stream, and these small launches would wait behind them
    {
        Timed tm(d, TSK_ROLE_OTHER, 2.0 * B * T * c.latent_dim * H, 2.0 * H * c.latent_dim + 4.0 * B * T * (c.latent_dim + H), st);
        const uint16_t *w_in = wptr<uint16_t>(d, "audio_input_proj.weight");
        const float *b_in = wptr<float>(d, "audio_input_proj.bias");
        e = latent_cm ? launch_proj_f32_cm(w_in, b_in, latent_d, T, B * T, c.latent_dim, H, d->lat, H, d->xf, st)
                      : launch_proj_f32(w_in, b_in, latent_d, c.latent_dim, B * T, c.latent_dim, H, d->lat, H, st);
        if (e != hipSuccess) return hip_fail(e, "input projection");
    }
    if ((e = hipMemcpyAsync(d->txt, text_d, sizeof(float) * B * St * H, hipMemcpyDeviceToDevice, st)) != hipSuccess)
        return hip_fail(e, "text copy");
    bool joined = true;
    if (!d->cur_sched) {
        if ((rc = run_conditioning(d, B, t_host, jmain, st))) return rc;
        joined = false;
    }
    auto join = [&]() -> int {
        if (joined) return TSK_OK;
        joined = true;
        return hipcheck(hipStreamWaitEvent(st, d->ev_join, 0), "join");
    };

    // streams: latent rows of this call first, text rows from the capacity offset
    const size_t cap = (size_t) c.max_batch * c.max_latent;
    StreamRun L, X;
    L.w = nullptr; L.x = d->lat; L.S = T; L.tok_off = 0; L.rope = 1;
    L.xn = d->xn; L.h = d->h; L.part = d->part; L.row_off = 0;
    X.w = nullptr; X.x = d->txt; X.S = St; X.tok_off = T; X.rope = 0;
    X.xn = d->xn + cap * H; X.h = d->h + cap * c.mlp_hidden; X.part = d->part + (size_t) KSPLIT_MAX * cap * H;
    X.row_off = (int64_t) cap;
    // joint blocks: LN -> QKV (+RMSNorm/RoPE/F16 epilogue) -> attention over the
    // concatenated tokens -> linear1 (split-K) -> residual + LN -> fc1 (+GELU)
    // -> fc2 (split-K, residual paid by the next LN); both streams per launch
    const int Nj = T + St;
    for (int i = 0; i < nj; ++i) {
        if (2 * i >= jmain && (rc = join())) return rc;
        L.w = &d->joint_lat[i];
        X.w = &d->joint_txt[i];
        StreamRun r2[2] = {L, X};
        if (d->q8) {
            if ((rc = block_q8(d, r2, 2, B, Nj, st))) return rc;
            L = r2[0];
            X = r2[1];
            continue;
        }
        if ((rc = run_ln(d, r2, 2, B, 0, st))) return rc;
        if ((rc = run_qkv(d, r2, 2, B, Nj, st))) return rc;
        if ((rc = attention(d, r2, 2, B, Nj, st))) return rc;
        if ((rc = run_out(d, r2, 2, B, Nj, st))) return rc;
        const int ns = r2[1].w->pre_only ? 1 : 2;
        if ((rc = run_ln(d, r2, ns, B, 1, st))) return rc;
        if ((rc = run_mlp(d, r2, ns, B, st))) return rc;
        L = r2[0];
        X = r2[1];
    }
    // fused blocks: the latent stream alone
    if ((rc = join())) return rc;
    for (int i = 0; i < c.fused_depth; ++i) {
        L.w = &d->fused[i];
        if (d->q8) {
            if ((rc = block_q8(d, &L, 1, B, T, st))) return rc;
            continue;
        }
        if ((rc = run_ln(d, &L, 1, B, 0, st))) return rc;
        if ((rc = run_qkv(d, &L, 1, B, T, st))) return rc;
        if ((rc = attention(d, &L, 1, B, T, st))) return rc;
        if ((rc = run_out(d, &L, 1, B, T, st))) return rc;
        if ((rc = run_ln(d, &L, 1, B, 1, st))) return rc;
        if ((rc = run_mlp(d, &L, 1, B, st))) return rc;
    }
    // final layer: last residual update + LN/modulate (f32, final adaLN shift/scale)
    // -> linear to latent_dim (f32 activations, fp32 accumulation)
    {
        const float *fmod = d->cur_sched ? d->cur_sched + d->sched_final : d->final_mod;
        LnGroup g;
        memset(&g, 0, sizeof(g));
        g.nstream = 1; g.H = H; g.eps = c.ln_eps; g.y_mode = LN_Y_F32;
        g.s[0] = ln_stream(L, B, H, d->cur_sched ? 0 : 2 * H, fmod, fmod + H, d->xf);
        Timed tm(d, TSK_ROLE_OTHER, 10.0 * B * T * H, 16.0 * B * T * H + 4.0 * L.pend_split * B * T * H, st);
        if ((e = launch_ln_group(g, st)) != hipSuccess) return hip_fail(e, "final ln");
    }
    Timed tm(d, TSK_ROLE_OTHER, 2.0 * B * T * H * c.latent_dim, 4.0 * B * T * H + 2.0 * H * c.latent_dim, st);
    e = launch_proj_f32(wptr<uint16_t>(d, "final_layer.linear.weight"), wptr<float>(d, "final_layer.linear.bias"), d->xf, H,
                        B * T, H, c.latent_dim, flow_d, c.latent_dim, st);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "final projection");
}

int check_forward_args(tsk_dit *d, int B, int T, const void *a, const void *t, const void *b, const void *f) {
    if (!d || !a || !t || !b || !f) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    if (B < 1 || B > d->cfg.max_batch) return fail(TSK_ERR_SHAPE, "B=%d outside [1, %d]", B, d->cfg.max_batch);
    if (T < 1 || T > d->cfg.max_latent) return fail(TSK_ERR_SHAPE, "T=%d outside [1, %d]", T, d->cfg.max_latent);
    return require_init();
}

}  // namespace

extern "C" int tsk_dit_forward_device(tsk_dit *d, int B, int T, const float *latent_d, const float *t_host,
                                      const float *text_d, float *flow_d, tsk_stream stream) {
    int rc = check_forward_args(d, B, T, latent_d, t_host, text_d, flow_d);
    if (rc) return rc;
    return forward_impl(d, B, T, latent_d, true, t_host, text_d, flow_d, (hipStream_t) stream);
}

extern "C" int tsk_dit_forward(tsk_dit *d, int B, int T, const float *latent, const float *t, const float *text,
                               float *flow, tsk_stream stream) {
    int rc = check_forward_args(d, B, T, latent, t, text, flow);
    if (rc) return rc;
    const tsk_dit_config &c = d->cfg;
    hipStream_t st = (hipStream_t) stream;
    // the host inputs go to the staging buffer allocated at create (B <= max_batch, T <= max_latent)
    const size_t nl = (size_t) B * T * c.latent_dim, nt = (size_t) B * c.text_seq * c.hidden;
    float *lat_d = d->in_stage, *txt_d = d->in_stage + nl;
    rc = hipcheck(hipMemcpyAsync(lat_d, latent, sizeof(float) * nl, hipMemcpyHostToDevice, st), "latent upload");
    if (!rc) rc = hipcheck(hipMemcpyAsync(txt_d, text, sizeof(float) * nt, hipMemcpyHostToDevice, st), "text upload");
    if (!rc) rc = forward_impl(d, B, T, lat_d, true, t, txt_d, d->flow, st);
    if (!rc) rc = hipcheck(hipMemcpyAsync(flow, d->flow, sizeof(float) * nl, hipMemcpyDeviceToHost, st), "flow download");
    // the pageable sources and destination are done with once the stream is
    (void) hipStreamSynchronize(st);
    if (!rc) rc = hipcheck(hipGetLastError(), "stream sync");
    return rc;
}

// ------------------------------------------------------------------ sampler
namespace {

// The sampler's t values are fixed by its step count (linspace(1, 0, steps + 1),
// mmdit.cpp:360-362) and the adaLN modulations depend on t alone, identically
// for the conditional and the unconditional row. They are computed for every
// step before the first one, 32 steps per batched pass, so each adaLN weight
// matrix is read once per 32 steps instead of once per step; every output is
// summed exactly as the per-call path sums it (the GEMV's summation order does
// not depend on its batch), so the schedule changes no result bit.
int build_schedule(tsk_dit *d, int steps, hipStream_t st) {
    const int H = d->cfg.hidden;
    const size_t R = d->sched_row;
    const int nchunk = (steps + 31) / 32;
    const int nj = d->njobs;                  // block + final-layer jobs; t_embed.0 / .2 follow
    const int per = nj + 2;
    hipError_t e;
    if (d->sched_cap < (size_t) steps * R) {
        if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail(e, "sync");
        if (d->sched) (void) hipFree(d->sched);
        d->sched = nullptr;
        d->sched_cap = 0;
        if (hipMalloc((void **) &d->sched, sizeof(float) * (size_t) steps * R) != hipSuccess)
            return fail(TSK_ERR_NOMEM, "hipMalloc conditioning schedule (%d steps)", steps);
        d->sched_cap = (size_t) steps * R;
    }
    if (!d->sched_act && hipMalloc((void **) &d->sched_act, sizeof(float) * 3 * 32 * H) != hipSuccess)
        return fail(TSK_ERR_NOMEM, "hipMalloc schedule activations");
    if (d->sched_jobs_cap < nchunk * per) {
        if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail(e, "sync");
        if (d->sched_jobs) (void) hipFree(d->sched_jobs);
        d->sched_jobs = nullptr;
        d->sched_jobs_cap = 0;
        if (hipMalloc((void **) &d->sched_jobs, sizeof(GemvJob) * nchunk * per) != hipSuccess)
            return fail(TSK_ERR_NOMEM, "hipMalloc schedule jobs");
        d->sched_jobs_cap = nchunk * per;
    }
    float *temb = d->sched_act, *hid = temb + 32 * H, *cvec = hid + 32 * H;
    std::vector<GemvJob> tab((size_t) nchunk * per);
    for (int ck = 0; ck < nchunk; ++ck) {
        GemvJob *t = tab.data() + (size_t) ck * per;
        float *row0 = d->sched + (size_t) ck * 32 * R;
        for (int j = 0; j < nj; ++j) {
            t[j] = d->jobs_host[j];
            t[j].x = cvec;
            t[j].out = row0 + d->jobs_sched_off[j];
            t[j].ld_out = (int64_t) R;
        }
        t[nj] = d->jobs_host[nj];
        t[nj].x = temb; t[nj].out = hid; t[nj].ld_out = H;
        t[nj + 1] = d->jobs_host[nj + 1];
        t[nj + 1].x = hid; t[nj + 1].out = cvec; t[nj + 1].ld_out = H;
    }
    // the table is read by kernels queued on st: copy it before any of them
    if ((e = hipStreamSynchronize(st)) != hipSuccess) return hip_fail(e, "sync");
    if ((e = hipMemcpy(d->sched_jobs, tab.data(), sizeof(GemvJob) * tab.size(), hipMemcpyHostToDevice)) != hipSuccess)
        return hip_fail(e, "hipMemcpy schedule jobs");
    const double wel = (double) R * H;   // adaLN weight elements
    Timed tm(d, TSK_ROLE_ADALN, 2.0 * steps * (wel + 2.0 * H * H), 2.0 * nchunk * (wel + 2.0 * H * H), st);
    for (int ck = 0; ck < nchunk; ++ck) {
        const int Bc = std::min(32, steps - 32 * ck);
        TimeVals tv;
        for (int b = 0; b < 32; ++b) tv.t[b] = b < Bc ? 1.0f - (float) (32 * ck + b) / (float) steps : 0.0f;
        const GemvJob *t = d->sched_jobs + (size_t) ck * per;
        if ((e = launch_timestep_embed(d->freq, tv, Bc, H, temb, st)) != hipSuccess) return hip_fail(e, "timestep embed");
        if ((e = launch_gemv_jobs(t + nj, 1, H, Bc, H, st)) != hipSuccess) return hip_fail(e, "t_embed.0");
        if ((e = launch_gemv_jobs(t + nj + 1, 1, H, Bc, H, st)) != hipSuccess) return hip_fail(e, "t_embed.2");
        if ((e = launch_gemv_jobs(t, nj, d->max_job_m, Bc, H, st)) != hipSuccess) return hip_fail(e, "adaln schedule");
    }
    return TSK_OK;
}

}  // namespace

extern "C" int tsk_dit_sample(tsk_dit *d, int T, const float *noise, const float *text_cond,
                              const float *text_uncond, int steps, float cfg_scale, float *out, float *flow0,
                              tsk_stream stream) {
    if (!d || !noise || !text_cond || !text_uncond || !out) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    if (d->cfg.max_batch < 2) return fail(TSK_ERR_SHAPE, "CFG needs max_batch >= 2");
    if (T < 1 || T > d->cfg.max_latent) return fail(TSK_ERR_SHAPE, "T=%d", T);
    if (steps < 1) return fail(TSK_ERR_INVALID_ARG, "steps=%d", steps);
    int rc = require_init();
    if (rc) return rc;
    const tsk_dit_config &c = d->cfg;
    hipStream_t st = (hipStream_t) stream;
    const size_t n = (size_t) T * c.latent_dim, nt = (size_t) c.text_seq * c.hidden;
    if (!d->s_x) {
        const size_t cap = (size_t) c.max_latent * c.latent_dim;
        hipError_t e = hipMalloc((void **) &d->s_x, sizeof(float) * cap * 6 + sizeof(float) * 2 * nt);
        if (e != hipSuccess) return fail(TSK_ERR_NOMEM, "hipMalloc sampler buffers");
        d->s_x2 = d->s_x + cap;
        d->s_flow2 = d->s_x + 3 * cap;
        d->s_flow0 = d->s_x + 5 * cap;
        d->s_text2 = d->s_x + 6 * cap;
    }
    // noise / out / flow0 are [latent_dim][T] (ne0 = T) as in ts_dit::sample;
    // the state on the device is token-major [T][latent_dim]
    const int L = c.latent_dim;
    std::vector<float> xt(n);
    for (int t = 0; t < T; ++t)
        for (int ch = 0; ch < L; ++ch) xt[(size_t) t * L + ch] = noise[(size_t) ch * T + t];
    if ((rc = hipcheck(hipMemcpyAsync(d->s_x, xt.data(), sizeof(float) * n, hipMemcpyHostToDevice, st), "noise"))) return rc;
    if ((rc = hipcheck(hipMemcpyAsync(d->s_x2, xt.data(), sizeof(float) * n, hipMemcpyHostToDevice, st), "noise"))) return rc;
    if ((rc = hipcheck(hipMemcpyAsync(d->s_x2 + n, xt.data(), sizeof(float) * n, hipMemcpyHostToDevice, st), "noise"))) return rc;
    if ((rc = hipcheck(hipMemcpyAsync(d->s_text2, text_cond, sizeof(float) * nt, hipMemcpyHostToDevice, st), "text"))) return rc;
    if ((rc = hipcheck(hipMemcpyAsync(d->s_text2 + nt, text_uncond, sizeof(float) * nt, hipMemcpyHostToDevice, st), "text"))) return rc;
    // xt is pageable host memory that ends with this call: let the stream consume it first
    if ((rc = hipcheck(hipStreamSynchronize(st), "input upload"))) return rc;
    // Tuning::dit_sched off computes the conditioning inside every step instead
    const bool use_sched = tuning().dit_sched;
    if (use_sched && (rc = build_schedule(d, steps, st))) return rc;
    struct SchedGuard {
        tsk_dit *d;
        ~SchedGuard() { d->cur_sched = nullptr; }
    } guard{d};
    for (int s = 0; s < steps; ++s) {
        // linspace(1, 0, steps + 1) (mmdit.cpp:360-362)
        const float t_curr = 1.0f - (float) s / (float) steps;
        const float t_prev = 1.0f - (float) (s + 1) / (float) steps;
        const float tt[2] = {t_curr, t_curr};
        d->cur_sched = use_sched ? d->sched + (size_t) s * d->sched_row : nullptr;
        if ((rc = forward_impl(d, 2, T, d->s_x2, false, tt, d->s_text2, d->s_flow2, st))) return rc;
        hipError_t e = launch_cfg_euler(d->s_flow2, (int64_t) n, cfg_scale, t_prev - t_curr, d->s_x, d->s_x2,
                                        s == 0 ? d->s_flow0 : nullptr, st);
        if (e != hipSuccess) return hip_fail(e, "cfg_euler");
    }
    std::vector<float> xo(n), f0(flow0 ? n : 0);
    if ((rc = hipcheck(hipMemcpyAsync(xo.data(), d->s_x, sizeof(float) * n, hipMemcpyDeviceToHost, st), "out"))) return rc;
    if (flow0 && (rc = hipcheck(hipMemcpyAsync(f0.data(), d->s_flow0, sizeof(float) * n, hipMemcpyDeviceToHost, st), "flow0")))
        return rc;
    if ((rc = hipcheck(hipStreamSynchronize(st), "sync"))) return rc;
    for (int t = 0; t < T; ++t)
        for (int ch = 0; ch < L; ++ch) {
            out[(size_t) ch * T + t] = xo[(size_t) t * L + ch];
            if (flow0) flow0[(size_t) ch * T + t] = f0[(size_t) t * L + ch];
        }
    return TSK_OK;
}

// ------------------------------------------------------------------ timing
extern "C" int tsk_dit_timing(tsk_dit *d, int enable) {
    if (!d) return fail(TSK_ERR_INVALID_ARG, "dit is NULL");
    if (enable) {
        for (auto &r : d->rt) { r.used = 0; r.launches = 0; r.flop = 0.0; r.bytes = 0.0; }
    }
    d->timing = enable != 0;
    return TSK_OK;
}

extern "C" int tsk_dit_timing_read(tsk_dit *d, int role, double *ms, int64_t *launches, double *flop, double *bytes) {
    if (!d || role < 0 || role >= TSK_ROLE_COUNT) return fail(TSK_ERR_INVALID_ARG, "role %d", role);
    RoleTiming &r = d->rt[role];
    double total = 0.0;
    if (r.used) {
        hipError_t e = hipEventSynchronize(r.ev[r.used - 1]);
        if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
        for (size_t i = 0; i + 1 < r.used; i += 2) {
            float m = 0.0f;
            e = hipEventElapsedTime(&m, r.ev[i], r.ev[i + 1]);
            if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
            total += m;
        }
    }
    if (ms) *ms = total;
    if (launches) *launches = r.launches;
    if (flop) *flop = r.flop;
    if (bytes) *bytes = r.bytes;
    return TSK_OK;
}
