// tsk_runtime.h — error reporting, per-stream workspaces and launch tuning of
// the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace tsk {

// record a message for tsk_last_error() and return status
int fail(int status, const char *fmt, ...);
int hip_fail(hipError_t e, const char *what);
// TSK_OK if tsk_init() was called
int require_init();

// Device scratch of at least `bytes` for one call enqueued on stream s: the
// buffer the caller bound to s with tsk_set_workspace (TSK_ERR_NOMEM if it is
// too small; never reallocated), or else one library-owned buffer per
// (device, stream), grown on demand. Growing waits for s only (the previous
// buffer can only be read by work queued on s) and reallocates; a caller that
// cannot allow that binds its own buffer, sized by tsk_workspace_size.
int workspace(hipStream_t s, size_t bytes, void **out);

// Launch-shape overrides for tuning sweeps and A/B tests, read from the
// environment by tsk_init (every call re-reads them) and never on a launch:
//   TSK_Q8_CFG    Q8_0 cooperative tile (2 = 64 x 64, 5 = 32 x 64; 0 = rule)
//   TSK_Q8_OLD    1: the 2 x 2-wave Q8_0 kernel for every shape
//   TSK_Q8_PAIR   0: the Q8_0 DiT's two streams as separate launches (A/B reference)
//   TSK_COOP_CFG  cooperative BF16 tile of the C-ABI GEMMs (0 = rule)
//   TSK_GEMM_CFG  DiT block GEMM tiles, one character per projection
//   TSK_ATTN_CFG  DiT attention launch shape (10 * key ranges + query blocks)
//   TSK_DIT_SCHED 0: the sampler computes its conditioning inside every step
//   TSK_LN_BLOCK  1: LayerNorm rows as one workgroup each (A/B reference)
//   TSK_GEMV_RW   rows per wave of the adaLN GEMVs (1, 2, 4)
//   TSK_F32_KSPLIT  most K slices of the reference graph's F32 convolutions (1 = unsplit, 2, 4, 8)
//   TSK_F32_TILE  F32 GEMM wave tiles, 10 * (16-row tiles) + 16-column tiles per wave (0 = by rule, 42, 44, 24, 22)
//   TSK_F32_T44   fewest 128 x 128 tiles for which the rule takes them (256)
//   TSK_GRAPH_KSPLIT / TSK_GRAPH_KSWG  most K slices of the reference graph's bf16 k3 convolutions (4) and
//                 the workgroup count (64 x 64 tiles x slices) they stop below (1536)
//   TSK_ATTN_Q8   Q8_0 driver: the attention writes linear1's Q8_0 activations itself (1), or f32 + quantize (0)
//   TSK_F32_DL / TSK_F32_DL_NS  F32 GEMM with direct global -> LDS loads (1, default; 0 = register staged)
//                 and its ring depth (2, default; 3)
//   TSK_F32_SPLIT reference graph: F32 matrices as three bf16 products (1, default; read when a model is
//                 created, which then holds the split copies) or fp32 MFMA products (0, read on every call)
//   TSK_SPLIT_WG  most 128 x 128 tiles times K slices of a split product's launch (512)
//   TSK_VAE_SPLIT VAE decoder: F32 products as three bf16 ones (1; read when a model is created, which then
//                 holds the split copies) or fp32 MFMA products (0, default; read on every call)
struct Tuning {
    int q8_cfg = 0;
    bool q8_old = false;
    bool q8_pair = true;                  // a joint block's two Q8_0 projections in one launch
    int coop_cfg = 0;
    int gemm_cfg[4] = {0, 0, 0, 0};
    int attn_cfg = 0;
    bool dit_sched = true;
    bool ln_block = false;
    int gemv_rw = 2;
    int f32_ksplit = 8;
    int f32_tile = 0;
    int f32_t44 = 256;
    int graph_ksplit = 4;
    int graph_ks_wg = 1536;
    int attn_q8 = 1;
    int attn_xcd = 1;
    int attn_vrows = 1;
    int q8_qkv_fused = 1;
    int f32_dl = 1;
    int f32_dl_ns = 2;
    int f32_split = 1;
    int split_wg = 512;
    int vae_split = 0;
    int ksplit_out = 2, ksplit_fc2 = 4;   // DiT split-K of linear1 / ffn.fc2 (1..4)
    bool ksplit_set = false;              // TSK_KSPLIT given: the two counts hold at every size
    int l2_prefetch = -1;                 // DiT LN kernels fetch the next projections' weights into L2:
                                          // -1 by activation rows, 0 never, 1 always
};
const Tuning &tuning();

// Dynamic LDS above the default per-workgroup limit, opted in for kernel
// `kern` on the current device before its launch (hipFuncSetAttribute acts
// per device). Thread-safe; a size is recorded only when the runtime accepted
// it, so a refused opt-in is retried on the next launch (runtimes that need
// no opt-in may refuse the call: the launch itself then decides).
void lds_opt_in(const void *kern, size_t bytes);
// LDS bytes a workgroup may allocate on the current device (cached per device)
size_t device_lds_per_block();

// Device limits read once per tsk_init for the current device.
struct DeviceInfo {
    int cus = 256;               // compute units
    size_t lds_per_block = 160 * 1024;   // bytes of LDS a workgroup may allocate
};
const DeviceInfo &device_info();

}  // namespace tsk
