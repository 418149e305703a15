// dit.cpp — MM-DiT step driver (placeholder entry points until the driver lands)
#include "../../include/tsk/tsk.h"
#include "tsk_runtime.h"

extern "C" void tsk_dit_default_config(tsk_dit_config *c) {
    if (!c) return;
    c->hidden = 1024; c->n_head = 16; c->head_dim = 64; c->depth = 21; c->fused_depth = 14;
    c->latent_dim = 64; c->text_seq = 77; c->mlp_hidden = 4096; c->mlp_kind = TSK_MLP_GELU_TANH;
    c->weight_type = TSK_TYPE_BF16; c->max_batch = 2; c->max_latent = 646;
    c->rope_theta = 10000.0f; c->t_max_period = 1.0f; c->ln_eps = 1e-5f; c->qk_eps = 1e-6f;
}
extern "C" int tsk_dit_create(const tsk_dit_config *, tsk_dit **out) { if (out) *out = nullptr; return tsk::fail(TSK_ERR_UNSUPPORTED, "dit driver not built"); }
extern "C" void tsk_dit_destroy(tsk_dit *) {}
extern "C" int tsk_dit_n_tensors(const tsk_dit *) { return 0; }
extern "C" int tsk_dit_tensor_info(const tsk_dit *, int, const char **, int64_t *) { return TSK_ERR_UNSUPPORTED; }
extern "C" int tsk_dit_set_tensor(tsk_dit *, const char *, const float *, int64_t) { return TSK_ERR_UNSUPPORTED; }
extern "C" int tsk_dit_forward(tsk_dit *, int, int, const float *, const float *, const float *, float *, tsk_stream) { return TSK_ERR_UNSUPPORTED; }
extern "C" int tsk_dit_forward_device(tsk_dit *, int, int, const float *, const float *, const float *, float *, tsk_stream) { return TSK_ERR_UNSUPPORTED; }
extern "C" int tsk_dit_sample(tsk_dit *, int, const float *, const float *, const float *, int, float, float *, float *, tsk_stream) { return TSK_ERR_UNSUPPORTED; }
