// tsk_api.cpp — C ABI of the gfx950 MM-DiT hot path (include/tsk/tsk.h).
// Every entry point validates its operands on the host and returns a
// tsk_status; nothing aborts. Kernels are enqueued on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <map>
#include <mutex>
#include <utility>

#include "../../include/tsk/tsk.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

using namespace tsk;

namespace tsk {

static thread_local char g_err[512];
static thread_local LaunchEvents g_launch_events = {nullptr, nullptr};

LaunchEvents &launch_events() { return g_launch_events; }

int fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(TSK_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// ---- per-process state: tuning, device limits and per-stream workspaces
namespace {
std::mutex g_mu;
int g_device = -1;
Tuning g_tuning;
DeviceInfo g_dev;
// one workspace per (device, stream): library-owned (grown on demand) or
// bound by the caller (external, never reallocated)
struct Workspace {
    void *ptr = nullptr;
    size_t size = 0;
    bool external = false;
};
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

int env_int(const char *name, int dflt) {
    const char *e = getenv(name);
    return e && *e ? atoi(e) : dflt;
}

void read_tuning() {
    Tuning t;
    t.q8_cfg = env_int("TSK_Q8_CFG", 0);
    t.q8_old = env_int("TSK_Q8_OLD", 0) != 0;
    t.q8_pair = env_int("TSK_Q8_PAIR", 1) != 0;
    t.coop_cfg = env_int("TSK_COOP_CFG", 0);
    t.attn_cfg = env_int("TSK_ATTN_CFG", 0);
    t.dit_sched = env_int("TSK_DIT_SCHED", 1) != 0;
    t.ln_block = env_int("TSK_LN_BLOCK", 0) != 0;
    t.gemv_rw = env_int("TSK_GEMV_RW", 2);
    t.f32_ksplit = env_int("TSK_F32_KSPLIT", 8);
    t.f32_tile = env_int("TSK_F32_TILE", 0);
    t.f32_t44 = env_int("TSK_F32_T44", 256);
    t.graph_ksplit = env_int("TSK_GRAPH_KSPLIT", 4);
    t.graph_ks_wg = env_int("TSK_GRAPH_KSWG", 1536);
    t.attn_q8 = env_int("TSK_ATTN_Q8", 1);
    t.attn_xcd = env_int("TSK_ATTN_XCD", 1);
    t.q8_qkv_fused = env_int("TSK_Q8_QKV_FUSED", 1);
    t.attn_vrows = env_int("TSK_ATTN_VROWS", 1);
    t.f32_dl = env_int("TSK_F32_DL", 1);
    t.f32_dl_ns = env_int("TSK_F32_DL_NS", 2);
    t.f32_split = env_int("TSK_F32_SPLIT", 1);
    t.split_wg = env_int("TSK_SPLIT_WG", 512);
    t.vae_split = env_int("TSK_VAE_SPLIT", 0);
    t.l2_prefetch = env_int("TSK_L2PF", -1);
    // two digits: split-K of linear1 and of ffn.fc2 in the DiT driver
    if (const char *ks = getenv("TSK_KSPLIT"))
        if ((ks[0] == '1' || ks[0] == '2' || ks[0] == '4') && (ks[1] == '1' || ks[1] == '2' || ks[1] == '4')) {
            t.ksplit_out = ks[0] - '0';
            t.ksplit_fc2 = ks[1] - '0';
            t.ksplit_set = true;
        }
    // one character per projection (qkv, out, fc1, fc2): 0-9, a-z = 10-35, A-Z = 36-61
    if (const char *gc = getenv("TSK_GEMM_CFG"))
        for (int i = 0; i < 4 && gc[i]; ++i)
            t.gemm_cfg[i] = gc[i] >= '0' && gc[i] <= '9'   ? gc[i] - '0'
                            : gc[i] >= 'a' && gc[i] <= 'z' ? gc[i] - 'a' + 10
                            : gc[i] >= 'A' && gc[i] <= 'Z' ? gc[i] - 'A' + 36
                                                           : 0;
    g_tuning = t;
}
}  // namespace

// Scratch of tsk_mul_mat_noalloc: one fixed array in every GPU's memory (it
// stays resident until the process ends). Host code never uses the array's
// name as an address: its device address comes from hipGetSymbolAddress,
// once per device with that device current.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t) TSK_MUL_MAT_NOALLOC_SCRATCH;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
namespace {
void *g_scratch_ptr[64];   // per device; nullptr until looked up

// the device address of `scratch` on device dev (current); g_mu held
int scratch_address_locked(int dev, void **out) {
    if (dev < 0 || dev >= 64) return fail(TSK_ERR_INVALID_ARG, "device id %d out of range", dev);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(TSK_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return TSK_OK;
}
}  // namespace

const Tuning &tuning() { return g_tuning; }
const DeviceInfo &device_info() { return g_dev; }

namespace {
std::mutex g_lds_mu;
std::map<std::pair<const void *, int>, size_t> g_lds_attr;   // (kernel, device) -> LDS bytes opted in
std::map<int, size_t> g_lds_dev;                             // device -> LDS bytes per workgroup
}  // namespace

void lds_opt_in(const void *kern, size_t bytes) {
    if (bytes <= 64 * 1024) return;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return;
    std::lock_guard<std::mutex> lk(g_lds_mu);
    size_t &have = g_lds_attr[{kern, dev}];
    if (bytes <= have) return;
    if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int) bytes) == hipSuccess) have = bytes;
    else (void) hipGetLastError();
}

size_t device_lds_per_block() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 64 * 1024;
    std::lock_guard<std::mutex> lk(g_lds_mu);
    auto it = g_lds_dev.find(dev);
    if (it != g_lds_dev.end()) return it->second;
    int v = 0;
    const size_t lim = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 0
                           ? (size_t) v : 64 * 1024;
    g_lds_dev[dev] = lim;
    return lim;
}

int require_init() {
    if (g_device < 0) return fail(TSK_ERR_NOT_INIT, "tsk_init() has not been called");
    return TSK_OK;
}

int workspace(hipStream_t s, size_t bytes, void **out) {
    *out = nullptr;
    if (!bytes) return TSK_OK;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_mu);
    Workspace &w = g_ws[std::make_pair(dev, s)];
    if (w.size < bytes) {
        if (w.external)
            return fail(TSK_ERR_NOMEM, "the workspace bound to this stream holds %zu bytes, the call needs %zu", w.size,
                        bytes);
        // only work queued on s reads this stream's buffer
        e = hipStreamSynchronize(s);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        if (w.ptr) (void) hipFree(w.ptr);
        w.ptr = nullptr;
        w.size = 0;
        const size_t sz = (bytes + 0xfffff) & ~(size_t) 0xfffff;
        e = hipMalloc(&w.ptr, sz);
        if (e != hipSuccess) return fail(TSK_ERR_NOMEM, "hipMalloc(%zu): %s", sz, hipGetErrorString(e));
        w.size = sz;
    }
    *out = w.ptr;
    return TSK_OK;
}

}  // namespace tsk

// ------------------------------------------------------------------ helpers
namespace {

int elt_size(int type) {
    switch (type) {
        case TSK_TYPE_F32: case TSK_TYPE_I32: return 4;
        case TSK_TYPE_F16: case TSK_TYPE_BF16: return 2;
        default: return 0;
    }
}

bool aligned(const void *p, size_t a) { return ((uintptr_t) p % a) == 0; }

int check_tensor(const tsk_tensor *t, const char *name) {
    if (!t) return fail(TSK_ERR_INVALID_ARG, "%s is NULL", name);
    if (!t->data) return fail(TSK_ERR_INVALID_ARG, "%s->data is NULL", name);
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] < 1) return fail(TSK_ERR_SHAPE, "%s->ne[%d] = %lld < 1", name, i, (long long) t->ne[i]);
    return TSK_OK;
}

// rows of ne[0] contiguous elements, row stride aligned to `row_align` bytes
int check_rows(const tsk_tensor *t, const char *name, size_t row_align) {
    const int es = elt_size(t->type);
    if (!es) return fail(TSK_ERR_TYPE, "%s: type %d not supported here", name, t->type);
    if (t->nb[0] != (size_t) es) return fail(TSK_ERR_STRIDE, "%s: nb[0] = %zu, rows must be contiguous", name, t->nb[0]);
    for (int i = 1; i < 4; ++i)
        if (t->ne[i] > 1 && t->nb[i] % row_align)
            return fail(TSK_ERR_ALIGN, "%s: nb[%d] = %zu not a multiple of %zu", name, i, t->nb[i], row_align);
    if (!aligned(t->data, row_align)) return fail(TSK_ERR_ALIGN, "%s: data not %zu-byte aligned", name, row_align);
    return TSK_OK;
}

View4 view(const tsk_tensor *t) {
    View4 v;
    v.data = t->data;
    v.type = t->type;
    for (int i = 0; i < 4; ++i) { v.ne[i] = t->ne[i]; v.nb[i] = (int64_t) t->nb[i]; }
    return v;
}

bool same_shape(const tsk_tensor *a, const tsk_tensor *b) {
    for (int i = 0; i < 4; ++i) if (a->ne[i] != b->ne[i]) return false;
    return true;
}

// b rows are uniformly strided over (ne1, ne2, ne3) -> one GEMM with N = ne1*ne2*ne3
bool rows_uniform(const tsk_tensor *t) {
    return (t->ne[2] == 1 || t->nb[2] == t->nb[1] * (size_t) t->ne[1]) &&
           (t->ne[3] == 1 || t->nb[3] == t->nb[2] * (size_t) t->ne[2]);
}

}  // namespace

// ------------------------------------------------------------------ library
extern "C" int tsk_init(int device) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= n) return fail(TSK_ERR_INVALID_ARG, "device %d of %d", device, n);
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    DeviceInfo di;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && v > 0) di.cus = v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess && v > 0)
        di.lds_per_block = (size_t) v;
    std::lock_guard<std::mutex> lk(g_mu);
    void *sp = nullptr;
    int rc = scratch_address_locked(device, &sp);
    if (rc) return rc;
    read_tuning();
    g_dev = di;
    g_device = device;
    return TSK_OK;
}

extern "C" int tsk_shutdown(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_device < 0) return TSK_OK;
    (void) hipDeviceSynchronize();
    for (auto &kv : g_ws)
        if (kv.second.ptr && !kv.second.external) (void) hipFree(kv.second.ptr);
    g_ws.clear();
    g_device = -1;
    return TSK_OK;
}

extern "C" int tsk_set_workspace(tsk_stream stream, void *ptr, size_t bytes) {
    int rc = require_init();
    if (rc) return rc;
    if (!ptr != !bytes) return fail(TSK_ERR_INVALID_ARG, "ptr and bytes must both be set or both be zero");
    if (ptr && ((uintptr_t) ptr & 255)) return fail(TSK_ERR_ALIGN, "workspace must be 256-byte aligned");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    hipStream_t s = (hipStream_t) stream;
    std::lock_guard<std::mutex> lk(g_mu);
    Workspace &w = g_ws[std::make_pair(dev, s)];
    if (w.ptr && !w.external) {
        // the library-owned buffer may still be read by work queued on s
        e = hipStreamSynchronize(s);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        (void) hipFree(w.ptr);
    }
    w.ptr = ptr;
    w.size = bytes;
    w.external = ptr != nullptr;
    return TSK_OK;
}

extern "C" int tsk_release_workspace(tsk_stream stream) {
    int rc = require_init();
    if (rc) return rc;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    hipStream_t s = (hipStream_t) stream;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_ws.find(std::make_pair(dev, s));
    if (it == g_ws.end()) return TSK_OK;
    if (it->second.ptr && !it->second.external) {
        e = hipStreamSynchronize(s);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        (void) hipFree(it->second.ptr);
    }
    g_ws.erase(it);
    return TSK_OK;
}

extern "C" const char *tsk_status_string(int s) {
    switch (s) {
        case TSK_OK: return "ok";
        case TSK_ERR_INVALID_ARG: return "invalid argument";
        case TSK_ERR_TYPE: return "unsupported type";
        case TSK_ERR_SHAPE: return "shape mismatch";
        case TSK_ERR_STRIDE: return "unsupported strides";
        case TSK_ERR_ALIGN: return "misaligned operand";
        case TSK_ERR_UNSUPPORTED: return "unsupported operation";
        case TSK_ERR_NOT_INIT: return "library not initialised";
        case TSK_ERR_HIP: return "HIP runtime error";
        case TSK_ERR_NOMEM: return "out of device memory";
        default: return "unknown status";
    }
}

extern "C" const char *tsk_last_error(void) { return g_err; }
extern "C" const char *tsk_version(void) { return "tsk 0.1 gfx950"; }

// ------------------------------------------------------------------ mul_mat
namespace {

int validate_mul_mat(const tsk_tensor *a, const tsk_tensor *b, const tsk_tensor *bias, const tsk_tensor *dst) {
    int rc;
    if ((rc = check_tensor(a, "a")) || (rc = check_tensor(b, "b")) || (rc = check_tensor(dst, "dst"))) return rc;
    if (bias && (rc = check_tensor(bias, "bias"))) return rc;
    const int64_t K = a->ne[0], M = a->ne[1];
    if (a->ne[2] != 1 || a->ne[3] != 1) return fail(TSK_ERR_UNSUPPORTED, "a must be 2-D (weights), got ne2=%lld ne3=%lld", (long long) a->ne[2], (long long) a->ne[3]);
    if (b->ne[0] != K) return fail(TSK_ERR_SHAPE, "b->ne[0]=%lld != K=%lld", (long long) b->ne[0], (long long) K);
    if (dst->ne[0] != M || dst->ne[1] != b->ne[1] || dst->ne[2] != b->ne[2] || dst->ne[3] != b->ne[3])
        return fail(TSK_ERR_SHAPE, "dst must be [M=%lld, %lld, %lld, %lld]", (long long) M, (long long) b->ne[1], (long long) b->ne[2], (long long) b->ne[3]);
    if (b->type != TSK_TYPE_F32 && b->type != TSK_TYPE_BF16) return fail(TSK_ERR_TYPE, "b must be F32 or BF16");
    if (dst->type != TSK_TYPE_F32 && dst->type != TSK_TYPE_BF16) return fail(TSK_ERR_TYPE, "dst must be F32 or BF16");
    if ((rc = check_rows(b, "b", 16)) || (rc = check_rows(dst, "dst", 16))) return rc;
    if (bias) {
        if (bias->type != TSK_TYPE_F32 || bias->ne[0] != M || bias->ne[1] * bias->ne[2] * bias->ne[3] != 1)
            return fail(TSK_ERR_SHAPE, "bias must be F32 [M]");
        if (bias->nb[0] != 4 || !aligned(bias->data, 16)) return fail(TSK_ERR_ALIGN, "bias must be contiguous, 16-byte aligned");
    }
    switch (a->type) {
        case TSK_TYPE_BF16:
            if (K % 8) return fail(TSK_ERR_SHAPE, "K=%lld must be a multiple of 8 for BF16", (long long) K);
            if ((rc = check_rows(a, "a", 16))) return rc;
            break;
        case TSK_TYPE_Q8_0:
            if (K % 32) return fail(TSK_ERR_SHAPE, "K=%lld must be a multiple of 32 for Q8_0", (long long) K);
            if (a->nb[0] != 34) return fail(TSK_ERR_STRIDE, "Q8_0 a->nb[0] must be 34 (block size)");
            if (a->nb[1] < (size_t) (K / 32) * 34) return fail(TSK_ERR_STRIDE, "Q8_0 rows overlap");
            if (b->type != TSK_TYPE_F32 && b->type != TSK_TYPE_BF16) return fail(TSK_ERR_TYPE, "b type");
            break;
        case TSK_TYPE_Q8_0_SPLIT:
            if (K % 32) return fail(TSK_ERR_SHAPE, "K=%lld must be a multiple of 32 for Q8_0", (long long) K);
            if (!aligned(a->data, 16)) return fail(TSK_ERR_ALIGN, "Q8_0_SPLIT data must be 16-byte aligned");
            break;
        case TSK_TYPE_F32:
            // vec_dot type F32: the activations stay fp32
            if (b->type != TSK_TYPE_F32) return fail(TSK_ERR_TYPE, "F32 weights need F32 b");
            if (K % 8) return fail(TSK_ERR_SHAPE, "K=%lld must be a multiple of 8 for F32", (long long) K);
            if ((rc = check_rows(a, "a", 16))) return rc;
            break;
        case TSK_TYPE_F16:
            return fail(TSK_ERR_UNSUPPORTED, "mul_mat with F16 weights is not implemented on gfx950 (F32, BF16, Q8_0)");
        default:
            return fail(TSK_ERR_TYPE, "weight type %d", a->type);
    }
    return TSK_OK;
}

}  // namespace

namespace {

// Scratch of one call: the workspace of its stream (tsk_set_workspace or the
// library's own), or a fixed region with a hard limit.
struct Scratch {
    hipStream_t s;
    void *fixed;
    size_t cap;
    int get(size_t bytes, void **out) const {
        if (!fixed) return workspace(s, bytes, out);
        if (bytes > cap)
            return fail(TSK_ERR_NOMEM, "the call needs %zu bytes of scratch, the limit is %zu", bytes, cap);
        *out = bytes ? fixed : nullptr;
        return TSK_OK;
    }
};

size_t align256(size_t n) { return (n + 255) & ~(size_t) 255; }

// How tsk_mul_mat runs a validated node, and the scratch it needs.
struct MulMatPlan {
    bool uni;            // rows of b and dst uniformly strided: one GEMM of Nslice rows
    int64_t nslices, Nslice;
    bool coop;           // BF16 weights on the cooperative tiles
    size_t cast_bytes;   // coop with f32 b: b rounded to bf16 rows
    size_t wbytes;       // Q8_0: the weights repacked into planes
    size_t act_bytes;    // Q8_0 / Q8_0_SPLIT: the quantized activation planes
    size_t bytes;        // total scratch
};

MulMatPlan plan_mul_mat(const tsk_tensor *a, const tsk_tensor *b, const tsk_tensor *dst) {
    MulMatPlan pl;
    memset(&pl, 0, sizeof(pl));
    const int64_t K = a->ne[0], M = a->ne[1];
    // slices of uniformly strided rows: one launch per (i2, i3) unless rows are uniform
    pl.uni = rows_uniform(b) && rows_uniform(dst);
    pl.nslices = pl.uni ? 1 : b->ne[2] * b->ne[3];
    pl.Nslice = pl.uni ? b->ne[1] * b->ne[2] * b->ne[3] : b->ne[1];
    pl.coop = a->type == TSK_TYPE_BF16 && pl.uni && M % 16 == 0 && K % 32 == 0 && a->nb[1] % 16 == 0;
    if (pl.coop && b->type == TSK_TYPE_F32) pl.cast_bytes = align256((size_t) (pl.Nslice * K) * 2);
    if (a->type == TSK_TYPE_Q8_0 || a->type == TSK_TYPE_Q8_0_SPLIT) {
        pl.wbytes = a->type == TSK_TYPE_Q8_0 ? align256(tsk_q8_0_split_nbytes(K, M)) : 0;
        pl.act_bytes = (((size_t) (pl.Nslice * K) + 15) & ~(size_t) 15) + sizeof(float) * (size_t) (pl.Nslice * (K / 32));
        pl.act_bytes = align256(pl.act_bytes);
    }
    pl.bytes = pl.cast_bytes + pl.wbytes + pl.act_bytes;
    return pl;
}

int mul_mat_impl(const tsk_tensor *a, const tsk_tensor *b, const tsk_tensor *bias, tsk_tensor *dst,
                 const Scratch &scr) {
    hipStream_t s = scr.s;
    const int64_t K = a->ne[0], M = a->ne[1];
    const int es_b = elt_size(b->type), es_d = elt_size(dst->type);
    const MulMatPlan pl = plan_mul_mat(a, b, dst);
    int rc;
    char *ws = nullptr;
    if ((rc = scr.get(pl.bytes, (void **) &ws))) return rc;
    const int64_t nslices = pl.nslices, Nslice = pl.Nslice;

    // BF16 weights with M % 16 == 0, K % 32 == 0 and uniformly strided rows:
    // the cooperative tiles of gemm_ks.hip on bf16 activation rows (f32 b is
    // rounded to bf16 into the scratch first: ggml's conversion of src1)
    if (pl.coop) {
        uint16_t *xb = nullptr;
        const int64_t N = Nslice;
        const int64_t ld_b = (int64_t) (b->nb[1] / es_b);
        if (b->type == TSK_TYPE_F32) {
            xb = (uint16_t *) ws;
            hipError_t e = launch_cast_rows_bf16((const float *) b->data, ld_b, 0, (int) std::min<int64_t>(N, 1 << 30), N,
                                                 (int) K, xb, s);
            if (e != hipSuccess) return hip_fail(e, "mul_mat input cast");
        }
        GemmGroup g;
        memset(&g, 0, sizeof(g));
        g.nprob = 1;
        GemmProblem &q = g.p[0];
        q.x = xb ? (const void *) xb : b->data;
        q.ld_x = xb ? K : ld_b;
        q.w = (const uint16_t *) a->data;
        q.ld_w = (int64_t) (a->nb[1] / 2);
        q.bias = bias ? (const float *) bias->data : nullptr;
        q.y = dst->data;
        q.ld_y = (int64_t) (dst->nb[1] / es_d);
        q.M = (int) M; q.N = (int) N; q.K = (int) K; q.splits = 1;
        hipError_t e = launch_gemm_coop(g, dst->type == TSK_TYPE_BF16 ? EPI_STORE_BF16 : EPI_STORE_F32, s);
        return e == hipSuccess ? TSK_OK : hip_fail(e, "mul_mat launch");
    }

    // Q8_0 weights: repack raw ggml blocks into planes in the scratch
    const int8_t *qw = nullptr;
    const uint16_t *dw = nullptr;
    if (a->type == TSK_TYPE_Q8_0 || a->type == TSK_TYPE_Q8_0_SPLIT) {
        if (a->type == TSK_TYPE_Q8_0) {
            hipError_t e = launch_q8_repack(a->data, (int64_t) a->nb[1], M, K, ws, s);
            if (e != hipSuccess) return hip_fail(e, "q8 repack");
            qw = (const int8_t *) ws;
        } else {
            qw = (const int8_t *) a->data;
        }
        dw = (const uint16_t *) ((const char *) qw + (size_t) (M * K));
    }

    for (int64_t sl = 0; sl < nslices; ++sl) {
        const int64_t i2 = sl % b->ne[2], i3 = sl / b->ne[2];
        GemmParams p;
        memset(&p, 0, sizeof(p));
        p.x = (const char *) b->data + i2 * b->nb[2] + i3 * b->nb[3];
        p.y = (char *) dst->data + i2 * dst->nb[2] + i3 * dst->nb[3];
        p.bias = bias ? (const float *) bias->data : nullptr;
        p.ld_x = (int64_t) (b->nb[1] / es_b);
        p.ld_y = (int64_t) (dst->nb[1] / es_d);
        p.M = (int) M;
        p.N = (int) Nslice;
        p.K = (int) K;
        p.x_f32 = b->type == TSK_TYPE_F32;
        p.y_bf16 = dst->type == TSK_TYPE_BF16;
        p.epi = EPI_STORE;
        p.rows_per_gate = 1;
        hipError_t e;
        if (a->type == TSK_TYPE_BF16) {
            p.w = a->data;
            p.ld_w = (int64_t) (a->nb[1] / 2);
            e = launch_gemm_bf16(p, s);
        } else if (a->type == TSK_TYPE_F32) {
            GemmProblem q;
            memset(&q, 0, sizeof(q));
            q.x = p.x; q.wf = (const float *) a->data; q.bias = p.bias; q.y = p.y;
            q.ld_x = p.ld_x; q.ld_w = (int64_t) (a->nb[1] / 4); q.ld_y = p.ld_y;
            q.M = p.M; q.N = p.N; q.K = p.K; q.splits = 1;
            e = launch_gemm_f32(q, p.y_bf16, s);
        } else {
            char *act = ws + pl.wbytes;
            int8_t *qx = (int8_t *) act;
            float *dx = (float *) (act + (((size_t) (Nslice * K) + 15) & ~(size_t) 15));
            e = launch_quantize_rows_q8(p.x, p.x_f32, p.ld_x, p.N, p.K, qx, dx, s);
            if (e != hipSuccess) return hip_fail(e, "q8 activation quantize");
            p.qw = qw;
            p.dw = dw;
            p.qx = qx;
            p.dx = dx;
            e = launch_gemm_q8(p, s);
        }
        if (e != hipSuccess) return hip_fail(e, "mul_mat launch");
    }
    return TSK_OK;
}

}  // namespace

extern "C" int tsk_mul_mat(const tsk_tensor *a, const tsk_tensor *b, const tsk_tensor *bias, tsk_tensor *dst,
                           tsk_stream stream) {
    int rc = validate_mul_mat(a, b, bias, dst);
    if (rc) return rc;
    if ((rc = require_init())) return rc;
    return mul_mat_impl(a, b, bias, dst, Scratch{(hipStream_t) stream, nullptr, 0});
}

extern "C" int tsk_mul_mat_noalloc(const tsk_tensor *a, const tsk_tensor *b, const tsk_tensor *bias, tsk_tensor *dst,
                                   tsk_stream stream) {
    int rc = validate_mul_mat(a, b, bias, dst);
    if (rc) return rc;
    if ((rc = require_init())) return rc;
    const size_t need = plan_mul_mat(a, b, dst).bytes;
    if (need > NOALLOC_SCRATCH_BYTES)
        return fail(TSK_ERR_NOMEM, "tsk_mul_mat_noalloc: the node needs %zu bytes of scratch, the fixed limit is %zu",
                    need, NOALLOC_SCRATCH_BYTES);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    void *sp = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if ((rc = scratch_address_locked(dev, &sp))) return rc;
    }
    return mul_mat_impl(a, b, bias, dst, Scratch{(hipStream_t) stream, sp, NOALLOC_SCRATCH_BYTES});
}

// ------------------------------------------------------------------ flash_attn_ext
namespace {

int validate_fa(const tsk_tensor *q, const tsk_tensor *k, const tsk_tensor *v, const tsk_tensor *mask,
                float scale, float max_bias, float softcap, int prec, const tsk_tensor *dst) {
    int rc;
    if ((rc = check_tensor(q, "q")) || (rc = check_tensor(k, "k")) || (rc = check_tensor(v, "v")) ||
        (rc = check_tensor(dst, "dst")))
        return rc;
    if (mask && (rc = check_tensor(mask, "mask"))) return rc;
    if (q->ne[0] != 64 || k->ne[0] != 64 || v->ne[0] != 64)
        return fail(TSK_ERR_UNSUPPORTED, "head dim must be 64 (got q %lld, k %lld, v %lld)", (long long) q->ne[0], (long long) k->ne[0], (long long) v->ne[0]);
    if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2] || k->ne[3] != v->ne[3])
        return fail(TSK_ERR_SHAPE, "k and v shapes differ");
    if (q->ne[3] != k->ne[3]) return fail(TSK_ERR_SHAPE, "batch of q and k differ");
    if (q->ne[2] % k->ne[2]) return fail(TSK_ERR_SHAPE, "q heads %lld not a multiple of kv heads %lld", (long long) q->ne[2], (long long) k->ne[2]);
    if (dst->ne[0] != 64 || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] || dst->ne[3] != q->ne[3])
        return fail(TSK_ERR_SHAPE, "dst must be [64, H, Nq, B] (ggml permuted result)");
    for (const tsk_tensor *t : {q, k, v})
        if (t->type != TSK_TYPE_F32 && t->type != TSK_TYPE_F16 && t->type != TSK_TYPE_BF16)
            return fail(TSK_ERR_TYPE, "q/k/v type %d", t->type);
    if (k->type != v->type) return fail(TSK_ERR_TYPE, "k and v must have the same type");
    if (dst->type != TSK_TYPE_F32 && dst->type != TSK_TYPE_BF16) return fail(TSK_ERR_TYPE, "dst type");
    if ((rc = check_rows(q, "q", 16)) || (rc = check_rows(k, "k", 16)) || (rc = check_rows(v, "v", 16)) ||
        (rc = check_rows(dst, "dst", 16)))
        return rc;
    if (mask) {
        if (mask->type != TSK_TYPE_F16 && mask->type != TSK_TYPE_F32) return fail(TSK_ERR_TYPE, "mask must be F16 or F32");
        if (mask->ne[0] < k->ne[1] || mask->ne[1] < q->ne[1])
            return fail(TSK_ERR_SHAPE, "mask must cover [Nkv, Nq]");
        if (q->ne[2] % mask->ne[2] || q->ne[3] % mask->ne[3]) return fail(TSK_ERR_SHAPE, "mask broadcast");
        if (mask->nb[0] != (size_t) elt_size(mask->type)) return fail(TSK_ERR_STRIDE, "mask rows must be contiguous");
        if (!aligned(mask->data, elt_size(mask->type))) return fail(TSK_ERR_ALIGN, "mask data alignment");
    }
    if (!(scale > 0.0f) || !(max_bias >= 0.0f) || !(softcap >= 0.0f) || softcap != softcap)
        return fail(TSK_ERR_INVALID_ARG, "scale must be > 0, max_bias and softcap >= 0");
    if (prec != TSK_PREC_DEFAULT && prec != TSK_PREC_F32) return fail(TSK_ERR_INVALID_ARG, "prec %d", prec);
    return TSK_OK;
}

// Nodes the MFMA 32x32 kernel of attn_dit.hip runs: head_dim 64 (checked by
// validate_fa), 16-bit K/V, one KV head per head, no mask / softcap / ALiBi,
// 16-byte aligned rows.
bool fa_fast_eligible(const tsk_tensor *q, const tsk_tensor *k, const tsk_tensor *v, const tsk_tensor *mask,
                      float max_bias, float softcap, const tsk_tensor *dst) {
    if (mask || max_bias != 0.0f || softcap != 0.0f) return false;
    if (k->type != TSK_TYPE_F16 && k->type != TSK_TYPE_BF16) return false;
    if (v->type != TSK_TYPE_F16 && v->type != TSK_TYPE_BF16) return false;
    if (k->ne[2] != q->ne[2] || k->ne[3] != q->ne[3]) return false;
    if (q->ne[1] > (1 << 24) || k->ne[1] > (1 << 24)) return false;
    const tsk_tensor *rows16[3] = {q, k, dst};
    for (const tsk_tensor *t : rows16) {
        if (!aligned(t->data, 16)) return false;
        for (int i = 1; i < 4; ++i)
            if (t->nb[i] % 16) return false;
    }
    return true;
}

// F16 V (the cast mmdit.cpp:90 makes) goes to the kernel as rows: 16-byte
// aligned rows (validate_fa) and a 31-bit byte range per (batch, head)
bool fa_v_rows(const tsk_tensor *k, const tsk_tensor *v) {
    if (v->type != TSK_TYPE_F16 || k->type != TSK_TYPE_F16 || !aligned(v->data, 16)) return false;
    for (int i = 1; i < 4; ++i)
        if (v->nb[i] % 16) return false;
    return v->nb[1] >= 128 && (int64_t) (v->ne[1] - 1) * (int64_t) v->nb[1] + 128 < ((int64_t) 1 << 31);
}

// scratch of the fast path: V transposed to fp16 [B * H][64][ldv] (none for V rows)
size_t fa_ws_bytes(const tsk_tensor *q, const tsk_tensor *k, const tsk_tensor *v, const tsk_tensor *mask,
                   float max_bias, float softcap, const tsk_tensor *dst) {
    if (!fa_fast_eligible(q, k, v, mask, max_bias, softcap, dst) || fa_v_rows(k, v)) return 0;
    const int64_t ldv = (k->ne[1] + 63) / 64 * 64;
    return align256((size_t) 2 * q->ne[3] * q->ne[2] * 64 * ldv);
}

}  // namespace

extern "C" int tsk_flash_attn_ext(const tsk_tensor *q, const tsk_tensor *k, const tsk_tensor *v,
                                  const tsk_tensor *mask, float scale, float max_bias, float logit_softcap, int prec,
                                  tsk_tensor *dst, tsk_stream stream) {
    int rc = validate_fa(q, k, v, mask, scale, max_bias, logit_softcap, prec, dst);
    if (rc) return rc;
    if ((rc = require_init())) return rc;
    if (fa_fast_eligible(q, k, v, mask, max_bias, logit_softcap, dst)) {
        // the MFMA 32x32 kernel: F16 V as rows, else V transposed to fp16 in
        // the workspace first
        const int Nkv = (int) k->ne[1], H = (int) q->ne[2], B = (int) q->ne[3];
        const int ldv = (Nkv + 63) / 64 * 64;
        hipStream_t st = (hipStream_t) stream;
        AttnFastParams f;
        memset(&f, 0, sizeof(f));
        hipError_t e;
        if (fa_v_rows(k, v)) {
            f.v = v->data; f.v_nb1 = v->nb[1]; f.v_nb2 = v->nb[2]; f.v_nb3 = v->nb[3];
            f.v_rows = 1;
        } else {
            void *ws = nullptr;
            if ((rc = workspace(st, fa_ws_bytes(q, k, v, mask, max_bias, logit_softcap, dst), &ws))) return rc;
            e = launch_vt_transpose(v->data, v->type == TSK_TYPE_BF16, (int64_t) v->nb[1], (int64_t) v->nb[2],
                                    (int64_t) v->nb[3], Nkv, H, B, (uint16_t *) ws, ldv, st);
            if (e != hipSuccess) return hip_fail(e, "flash_attn_ext V transpose");
            f.vt = (const uint16_t *) ws;
        }
        f.q = q->data; f.k = k->data; f.o = dst->data;
        f.q_type = q->type; f.k_bf16 = k->type == TSK_TYPE_BF16; f.out_bf16 = dst->type == TSK_TYPE_BF16;
        f.Nq = (int) q->ne[1]; f.Nkv = Nkv; f.H = H; f.B = B;
        f.q_nb1 = q->nb[1]; f.q_nb2 = q->nb[2]; f.q_nb3 = q->nb[3];
        f.k_nb1 = k->nb[1]; f.k_nb2 = k->nb[2]; f.k_nb3 = k->nb[3];
        f.vt_bh = (int64_t) 64 * ldv;
        f.ldv = ldv;
        f.o_nb1 = dst->nb[1]; f.o_nb2 = dst->nb[2]; f.o_nb3 = dst->nb[3];
        f.c = scale * 1.4426950408889634f;
        f.force_cfg = tuning().attn_cfg;
        e = launch_attn_fast(f, st);
        if (e != hipSuccess) return hip_fail(e, "flash_attn_ext launch");
        return TSK_OK;
    }
    AttnParams p;
    memset(&p, 0, sizeof(p));
    p.q = q->data; p.k = k->data; p.v = v->data; p.o = dst->data;
    p.mask = mask ? mask->data : nullptr;
    p.q_type = q->type; p.kv_type = k->type;
    p.out_bf16 = dst->type == TSK_TYPE_BF16;
    p.mask_f16 = mask ? mask->type == TSK_TYPE_F16 : 1;
    p.Nq = (int) q->ne[1]; p.Nkv = (int) k->ne[1]; p.H = (int) q->ne[2]; p.Hkv = (int) k->ne[2]; p.B = (int) q->ne[3];
    p.q_nb1 = q->nb[1]; p.q_nb2 = q->nb[2]; p.q_nb3 = q->nb[3];
    p.k_nb1 = k->nb[1]; p.k_nb2 = k->nb[2]; p.k_nb3 = k->nb[3];
    p.v_nb1 = v->nb[1]; p.v_nb2 = v->nb[2]; p.v_nb3 = v->nb[3];
    if (mask) {
        p.m_nb1 = mask->nb[1]; p.m_nb2 = mask->nb[2]; p.m_nb3 = mask->nb[3];
        p.m_ne2 = (int) mask->ne[2]; p.m_ne3 = (int) mask->ne[3];
    } else {
        p.m_ne2 = p.m_ne3 = 1;
    }
    p.o_nb1 = dst->nb[1]; p.o_nb2 = dst->nb[2]; p.o_nb3 = dst->nb[3];
    p.softcap = logit_softcap;
    p.scale = logit_softcap != 0.0f ? scale / logit_softcap : scale;
    p.max_bias = max_bias;
    p.n_head_log2 = 1u << (uint32_t) floorf(log2f((float) p.H));
    p.m0 = powf(2.0f, -(max_bias) / (float) p.n_head_log2);
    p.m1 = powf(2.0f, -(max_bias / 2.0f) / (float) p.n_head_log2);
    hipError_t e = launch_attention(p, (hipStream_t) stream);
    if (e != hipSuccess) return hip_fail(e, "flash_attn_ext launch");
    return TSK_OK;
}

// ------------------------------------------------------------------ RMS norm -> Q8_0
namespace {

int check_w(const tsk_tensor *w, int64_t n);

int validate_rms_norm_q8(const tsk_tensor *x, const tsk_tensor *w, const tsk_tensor *dst) {
    int rc;
    if ((rc = check_tensor(x, "x")) || (rc = check_tensor(dst, "dst"))) return rc;
    if ((rc = check_w(w, x->ne[0]))) return rc;
    if (x->type != TSK_TYPE_F32 || dst->type != TSK_TYPE_Q8_0) return fail(TSK_ERR_TYPE, "x F32 -> dst Q8_0");
    if (!same_shape(x, dst)) return fail(TSK_ERR_SHAPE, "x and dst shapes differ");
    const int64_t n = x->ne[0];
    if (n != 1024 && n != 2048 && n != 4096)
        return fail(TSK_ERR_UNSUPPORTED, "rows of %lld (1024, 2048 or 4096 elements)", (long long) n);
    if ((rc = check_rows(x, "x", 16))) return rc;
    if (!aligned(w->data, 16)) return fail(TSK_ERR_ALIGN, "w must be 16-byte aligned");
    if (dst->nb[0] != 34 || dst->nb[1] < (size_t) (n / 32) * 34) return fail(TSK_ERR_STRIDE, "dst Q8_0 rows");
    if (!rows_uniform(x) || !rows_uniform(dst)) return fail(TSK_ERR_STRIDE, "rows must be uniformly strided");
    return TSK_OK;
}

size_t rms_norm_q8_ws_bytes(const tsk_tensor *x) {
    const size_t rows = (size_t) (x->ne[1] * x->ne[2] * x->ne[3]), n = (size_t) x->ne[0];
    return align256(rows * n) + align256(rows * (n / 32) * sizeof(float));
}

}  // namespace

extern "C" int tsk_rms_norm_q8_0(const tsk_tensor *x, const tsk_tensor *w, float eps, tsk_tensor *dst,
                                 tsk_stream stream) {
    int rc = validate_rms_norm_q8(x, w, dst);
    if (rc) return rc;
    if (!(eps >= 0.0f)) return fail(TSK_ERR_INVALID_ARG, "eps");
    if ((rc = require_init())) return rc;
    hipStream_t s = (hipStream_t) stream;
    const int64_t rows = x->ne[1] * x->ne[2] * x->ne[3], n = x->ne[0];
    char *ws = nullptr;
    if ((rc = workspace(s, rms_norm_q8_ws_bytes(x), (void **) &ws))) return rc;
    int8_t *qx = (int8_t *) ws;
    float *dx = (float *) (ws + align256((size_t) (rows * n)));
    hipError_t e = launch_rms_norm_q8((const float *) x->data, (int64_t) (x->nb[1] / 4), (const float *) w->data, eps,
                                      qx, dx, rows, (int) n, s);
    if (e == hipSuccess) e = launch_q8_planes_to_blocks(qx, dx, rows, n, dst->data, (int64_t) dst->nb[1], s);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "rms_norm_q8 launch");
}

// ------------------------------------------------------------------ T5 attention
extern "C" int tsk_t5_attention(const tsk_tensor *q, const tsk_tensor *k, const tsk_tensor *v,
                                const tsk_tensor *rel_lut, const uint8_t *key_valid, float scale, tsk_tensor *dst,
                                tsk_stream stream) {
    int rc;
    if ((rc = check_tensor(q, "q")) || (rc = check_tensor(k, "k")) || (rc = check_tensor(v, "v")) ||
        (rc = check_tensor(rel_lut, "rel_lut")) || (rc = check_tensor(dst, "dst")))
        return rc;
    if (!key_valid) return fail(TSK_ERR_INVALID_ARG, "key_valid is NULL");
    for (const tsk_tensor *t : {q, k, v, rel_lut, (const tsk_tensor *) dst})
        if (t->type != TSK_TYPE_F32) return fail(TSK_ERR_TYPE, "q, k, v, rel_lut and dst must be F32");
    const int64_t n = q->ne[1], H = q->ne[2];
    if (q->ne[0] != 64 || !same_shape(q, k) || !same_shape(q, v) || q->ne[3] != 1)
        return fail(TSK_ERR_SHAPE, "q, k, v must be [64, n, H, 1]");
    if (dst->ne[0] != 64 || dst->ne[1] != H || dst->ne[2] != n || dst->ne[3] != 1)
        return fail(TSK_ERR_SHAPE, "dst must be [64, H, n, 1]");
    const int64_t nl = rel_lut->ne[0];
    if (nl % 2 == 0 || (nl + 1) / 2 < n || rel_lut->ne[1] != H || rel_lut->ne[2] * rel_lut->ne[3] != 1)
        return fail(TSK_ERR_SHAPE, "rel_lut must be [2 n_max - 1, H] with n_max >= n = %lld", (long long) n);
    if (rel_lut->nb[0] != 4 || rel_lut->nb[1] % 4 || !aligned(rel_lut->data, 4))
        return fail(TSK_ERR_STRIDE, "rel_lut rows must be contiguous");
    if ((rc = check_rows(q, "q", 16)) || (rc = check_rows(k, "k", 16)) || (rc = check_rows(v, "v", 16)) ||
        (rc = check_rows(dst, "dst", 16)))
        return rc;
    if (!(scale > 0.0f)) return fail(TSK_ERR_INVALID_ARG, "scale must be > 0");
    if ((rc = require_init())) return rc;
    AttnParams p;
    memset(&p, 0, sizeof(p));
    p.q = q->data; p.k = k->data; p.v = v->data; p.o = dst->data;
    p.q_type = p.kv_type = TSK_TYPE_F32;
    p.Nq = p.Nkv = (int) n; p.H = p.Hkv = (int) H; p.B = 1;
    p.q_nb1 = q->nb[1]; p.q_nb2 = q->nb[2]; p.q_nb3 = q->nb[3];
    p.k_nb1 = k->nb[1]; p.k_nb2 = k->nb[2]; p.k_nb3 = k->nb[3];
    p.v_nb1 = v->nb[1]; p.v_nb2 = v->nb[2]; p.v_nb3 = v->nb[3];
    p.m_ne2 = p.m_ne3 = 1;
    p.o_nb1 = dst->nb[1]; p.o_nb2 = dst->nb[2]; p.o_nb3 = dst->nb[3];
    p.scale = scale;
    p.n_head_log2 = 1u << (uint32_t) floorf(log2f((float) H));
    p.m0 = p.m1 = 1.0f;
    p.rel_lut = (const float *) rel_lut->data;
    p.rel_nh = (int64_t) (rel_lut->nb[1] / 4);
    p.rel_off = (int) ((nl - 1) / 2);
    p.key_valid = key_valid;
    hipError_t e = launch_attention(p, (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "t5 attention launch");
}

// ------------------------------------------------------------------ norms / rope
namespace {

int check_unary(const tsk_tensor *x, const tsk_tensor *dst) {
    int rc;
    if ((rc = check_tensor(x, "x")) || (rc = check_tensor(dst, "dst"))) return rc;
    if (!same_shape(x, dst)) return fail(TSK_ERR_SHAPE, "x and dst shapes differ");
    for (const tsk_tensor *t : {x, dst})
        if (t->type != TSK_TYPE_F32 && t->type != TSK_TYPE_BF16) return fail(TSK_ERR_TYPE, "F32 or BF16 only");
    if ((rc = check_rows(x, "x", elt_size(x->type))) || (rc = check_rows(dst, "dst", elt_size(dst->type)))) return rc;
    return TSK_OK;
}

int check_w(const tsk_tensor *w, int64_t n) {
    int rc;
    if ((rc = check_tensor(w, "w"))) return rc;
    if (w->type != TSK_TYPE_F32 || w->ne[0] != n || w->ne[1] * w->ne[2] * w->ne[3] != 1 || w->nb[0] != 4)
        return fail(TSK_ERR_SHAPE, "w must be contiguous F32 [%lld]", (long long) n);
    return TSK_OK;
}

int check_pos(const tsk_tensor *pos, const tsk_tensor *x) {
    int rc;
    if ((rc = check_tensor(pos, "pos"))) return rc;
    if (pos->type != TSK_TYPE_I32 || pos->ne[0] != x->ne[2] || pos->nb[0] != 4)
        return fail(TSK_ERR_SHAPE, "pos must be contiguous I32 [ne2 of x = %lld]", (long long) x->ne[2]);
    return TSK_OK;
}

}  // namespace

extern "C" int tsk_rms_norm_mul(const tsk_tensor *x, const tsk_tensor *w, float eps, tsk_tensor *dst, tsk_stream stream) {
    int rc;
    if ((rc = check_unary(x, dst))) return rc;
    if (w && (rc = check_w(w, x->ne[0]))) return rc;
    if (!(eps >= 0.0f)) return fail(TSK_ERR_INVALID_ARG, "eps");
    if ((rc = require_init())) return rc;
    hipError_t e = launch_rms_norm_mul(view(x), w ? (const float *) w->data : nullptr, eps, view(dst), (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "rms_norm launch");
}

extern "C" int tsk_norm(const tsk_tensor *x, float eps, tsk_tensor *dst, tsk_stream stream) {
    int rc;
    if ((rc = check_unary(x, dst))) return rc;
    if (!(eps >= 0.0f)) return fail(TSK_ERR_INVALID_ARG, "eps");
    if ((rc = require_init())) return rc;
    hipError_t e = launch_norm(view(x), eps, view(dst), (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "norm launch");
}

extern "C" int tsk_rope_ext(const tsk_tensor *x, const tsk_tensor *pos, int n_dims, int mode, float freq_base,
                            float freq_scale, float ext_factor, float attn_factor, tsk_tensor *dst, tsk_stream stream) {
    int rc;
    if ((rc = check_unary(x, dst)) || (rc = check_pos(pos, x))) return rc;
    if (mode != TSK_ROPE_TYPE_NORMAL) return fail(TSK_ERR_UNSUPPORTED, "rope mode %d (NORMAL only)", mode);
    if (ext_factor != 0.0f || attn_factor != 1.0f) return fail(TSK_ERR_UNSUPPORTED, "ext_factor must be 0, attn_factor 1");
    if (n_dims <= 0 || (n_dims & 1) || n_dims > x->ne[0] || n_dims > 128) return fail(TSK_ERR_INVALID_ARG, "n_dims %d", n_dims);
    if (!(freq_base > 0.0f)) return fail(TSK_ERR_INVALID_ARG, "freq_base");
    if ((rc = require_init())) return rc;
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    hipError_t e = launch_rope(view(x), (const int32_t *) pos->data, n_dims, theta_scale, freq_scale, view(dst),
                               (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "rope launch");
}

extern "C" int tsk_qk_norm_rope(const tsk_tensor *x, const tsk_tensor *w, const tsk_tensor *pos, float eps, int n_dims,
                                float freq_base, float freq_scale, tsk_tensor *dst, tsk_stream stream) {
    int rc;
    if ((rc = check_unary(x, dst)) || (rc = check_w(w, 64))) return rc;
    if (x->ne[0] != 64) return fail(TSK_ERR_UNSUPPORTED, "head dim must be 64");
    if (pos && (rc = check_pos(pos, x))) return rc;
    if (pos && (n_dims <= 0 || (n_dims & 1) || n_dims > 64)) return fail(TSK_ERR_INVALID_ARG, "n_dims %d", n_dims);
    if (!(eps >= 0.0f) || (pos && !(freq_base > 0.0f))) return fail(TSK_ERR_INVALID_ARG, "eps / freq_base");
    if ((rc = require_init())) return rc;
    const float theta_scale = pos ? powf(freq_base, -2.0f / (float) n_dims) : 1.0f;
    hipError_t e = launch_qk_norm_rope(view(x), (const float *) w->data, pos ? (const int32_t *) pos->data : nullptr,
                                       eps, n_dims, theta_scale, freq_scale, view(dst), (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "qk_norm_rope launch");
}

// ------------------------------------------------------------------ Q8_0
extern "C" size_t tsk_q8_0_split_nbytes(int64_t K, int64_t M) {
    if (K <= 0 || M <= 0 || K % 32) return 0;
    return (size_t) (K * M) + 2 * (size_t) (M * (K / 32));
}

extern "C" int tsk_q8_0_quantize(const tsk_tensor *x, tsk_tensor *dst, tsk_stream stream) {
    int rc;
    if ((rc = check_tensor(x, "x")) || (rc = check_tensor(dst, "dst"))) return rc;
    if (x->type != TSK_TYPE_F32 || dst->type != TSK_TYPE_Q8_0) return fail(TSK_ERR_TYPE, "x F32 -> dst Q8_0");
    if (!same_shape(x, dst)) return fail(TSK_ERR_SHAPE, "shapes differ");
    if (x->ne[0] % 32) return fail(TSK_ERR_SHAPE, "ne0 %% 32 != 0");
    if ((rc = check_rows(x, "x", 4))) return rc;
    if (dst->nb[0] != 34) return fail(TSK_ERR_STRIDE, "dst nb[0] must be 34");
    if (!rows_uniform(x) || !rows_uniform(dst)) return fail(TSK_ERR_STRIDE, "rows must be uniformly strided");
    if ((rc = require_init())) return rc;
    const int64_t rows = x->ne[1] * x->ne[2] * x->ne[3];
    hipError_t e = launch_q8_quantize_blocks((const float *) x->data, (int64_t) (x->nb[1] / 4), rows, x->ne[0],
                                             dst->data, (int64_t) dst->nb[1], (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "q8 quantize launch");
}

extern "C" int tsk_q8_0_dequantize(const tsk_tensor *x, tsk_tensor *dst, tsk_stream stream) {
    int rc;
    if ((rc = check_tensor(x, "x")) || (rc = check_tensor(dst, "dst"))) return rc;
    if ((x->type != TSK_TYPE_Q8_0 && x->type != TSK_TYPE_Q8_0_SPLIT) || dst->type != TSK_TYPE_F32)
        return fail(TSK_ERR_TYPE, "x Q8_0/Q8_0_SPLIT -> dst F32");
    if (!same_shape(x, dst)) return fail(TSK_ERR_SHAPE, "shapes differ");
    if (x->ne[0] % 32) return fail(TSK_ERR_SHAPE, "ne0 %% 32 != 0");
    if ((rc = check_rows(dst, "dst", 4))) return rc;
    if (!rows_uniform(dst)) return fail(TSK_ERR_STRIDE, "dst rows must be uniformly strided");
    const bool split = x->type == TSK_TYPE_Q8_0_SPLIT;
    if (!split && (x->nb[0] != 34 || !rows_uniform(x))) return fail(TSK_ERR_STRIDE, "Q8_0 strides");
    if ((rc = require_init())) return rc;
    const int64_t rows = x->ne[1] * x->ne[2] * x->ne[3];
    hipError_t e = launch_q8_dequantize(x->data, split, rows, x->ne[0], split ? 0 : (int64_t) x->nb[1],
                                        (float *) dst->data, (int64_t) (dst->nb[1] / 4), (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "q8 dequantize launch");
}

extern "C" int tsk_q8_0_repack(const tsk_tensor *src, tsk_tensor *dst, tsk_stream stream) {
    int rc;
    if ((rc = check_tensor(src, "src")) || (rc = check_tensor(dst, "dst"))) return rc;
    if (src->type != TSK_TYPE_Q8_0 || dst->type != TSK_TYPE_Q8_0_SPLIT) return fail(TSK_ERR_TYPE, "Q8_0 -> Q8_0_SPLIT");
    if (!same_shape(src, dst) || src->ne[2] * src->ne[3] != 1) return fail(TSK_ERR_SHAPE, "2-D Q8_0 of equal shape");
    if (src->ne[0] % 32 || src->nb[0] != 34) return fail(TSK_ERR_STRIDE, "Q8_0 layout");
    if (!aligned(dst->data, 16)) return fail(TSK_ERR_ALIGN, "dst 16-byte alignment");
    if ((rc = require_init())) return rc;
    hipError_t e = launch_q8_repack(src->data, (int64_t) src->nb[1], src->ne[1], src->ne[0], dst->data, (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "q8 repack launch");
}

// ------------------------------------------------------------------ convolution / SwiGLU
namespace {

int64_t conv_out_len(int64_t IW, int64_t KW, int s0, int p0, int d0) {
    return (IW + 2 * (int64_t) p0 - (int64_t) d0 * (KW - 1) - 1) / s0 + 1;
}

bool contiguous(const tsk_tensor *t) {
    size_t nb = (size_t) elt_size(t->type);
    for (int i = 0; i < 4; ++i) {
        if (t->ne[i] > 1 && t->nb[i] != nb) return false;
        nb *= (size_t) t->ne[i];
    }
    return true;
}

// conv kernel [KW, IC, OC] read in place by the GEMM: rows of K = KW * IC in
// kw-major order, 16-B aligned
bool kw_major(const tsk_tensor *w) {
    const size_t es = (size_t) elt_size(w->type);
    return (w->ne[0] == 1 || w->nb[0] == (size_t) w->ne[1] * es) && (w->ne[1] == 1 || w->nb[1] == es) &&
           (w->ne[2] == 1 || (w->nb[2] % 16 == 0 && w->nb[2] >= (size_t) (w->ne[0] * w->ne[1]) * es)) &&
           aligned(w->data, 16);
}

int check_conv_weight(const tsk_tensor *w, const char *name) {
    int rc;
    if ((rc = check_tensor(w, name))) return rc;
    if (w->type != TSK_TYPE_BF16 && w->type != TSK_TYPE_F32)
        return fail(TSK_ERR_TYPE, "%s: conv kernels are BF16 or F32 (type %d)", name, w->type);
    if (w->ne[3] != 1) return fail(TSK_ERR_SHAPE, "%s must be [KW, IC, OC]", name);
    const size_t es = (size_t) elt_size(w->type);
    for (int i = 0; i < 3; ++i)
        if (w->nb[i] % es) return fail(TSK_ERR_STRIDE, "%s: nb[%d] not a multiple of the element size", name, i);
    if (!aligned(w->data, es)) return fail(TSK_ERR_ALIGN, "%s: data alignment", name);
    return TSK_OK;
}

// channels-fastest activations [C, S, B, 1]
int check_conv_act(const tsk_tensor *t, const char *name) {
    int rc;
    if ((rc = check_tensor(t, name))) return rc;
    if (t->type != TSK_TYPE_F32 && t->type != TSK_TYPE_BF16) return fail(TSK_ERR_TYPE, "%s: F32 or BF16", name);
    if (t->ne[3] != 1) return fail(TSK_ERR_SHAPE, "%s must be [C, S, B, 1]", name);
    return check_rows(t, name, 16);
}

int validate_conv(const tsk_tensor *w, const tsk_tensor *bias, const tsk_tensor *x, int s0, int p0, int d0,
                  const tsk_tensor *dst) {
    int rc;
    if ((rc = check_conv_weight(w, "w")) || (rc = check_conv_act(x, "x")) || (rc = check_conv_act(dst, "dst")))
        return rc;
    if (bias && (rc = check_tensor(bias, "bias"))) return rc;
    const int64_t KW = w->ne[0], IC = w->ne[1], OC = w->ne[2];
    if (x->ne[0] != IC) return fail(TSK_ERR_SHAPE, "x->ne[0]=%lld != IC=%lld", (long long) x->ne[0], (long long) IC);
    if (IC % 8) return fail(TSK_ERR_SHAPE, "IC=%lld must be a multiple of 8", (long long) IC);
    if (w->type == TSK_TYPE_F32 && x->type != TSK_TYPE_F32) return fail(TSK_ERR_TYPE, "F32 kernels need F32 x");
    if (s0 < 1 || d0 < 1 || p0 < 0) return fail(TSK_ERR_INVALID_ARG, "stride %d, padding %d, dilation %d", s0, p0, d0);
    const int64_t OW = conv_out_len(x->ne[1], KW, s0, p0, d0);
    if (OW < 1) return fail(TSK_ERR_SHAPE, "output length %lld < 1", (long long) OW);
    if (dst->ne[0] != OC || dst->ne[1] != OW || dst->ne[2] != x->ne[2])
        return fail(TSK_ERR_SHAPE, "dst must be [OC=%lld, OW=%lld, B=%lld, 1]", (long long) OC, (long long) OW,
                    (long long) x->ne[2]);
    if (!rows_uniform(dst)) return fail(TSK_ERR_STRIDE, "dst rows must be uniformly strided");
    if (KW * IC > (1 << 30) || OW * x->ne[2] > (1 << 30) || x->ne[1] > (1 << 30))
        return fail(TSK_ERR_SHAPE, "conv too large");
    if (bias) {
        if (bias->type != TSK_TYPE_F32 || bias->ne[0] != OC || bias->ne[1] * bias->ne[2] * bias->ne[3] != 1)
            return fail(TSK_ERR_SHAPE, "bias must be F32 [OC]");
        if (bias->nb[0] != 4 || !aligned(bias->data, 16)) return fail(TSK_ERR_ALIGN, "bias must be contiguous, 16-byte aligned");
    }
    return TSK_OK;
}

// bytes a kw-major copy of w needs in scratch (0 if w is used in place)
size_t conv_pack_bytes(const tsk_tensor *w) {
    return kw_major(w) ? 0 : align256((size_t) (w->ne[0] * w->ne[1] * w->ne[2]) * (size_t) elt_size(w->type));
}

// the kw-major rows of w: in place, or packed into *scratch (advanced)
int conv_weight_rows(const tsk_tensor *w, char **scratch, const void **rows, int64_t *ld, hipStream_t s) {
    const int es = elt_size(w->type);
    if (kw_major(w)) {
        *rows = w->data;
        *ld = w->ne[2] > 1 ? (int64_t) (w->nb[2] / es) : w->ne[0] * w->ne[1];
        return TSK_OK;
    }
    hipError_t e = launch_conv_pack(w->data, es, (int64_t) (w->nb[0] / es), (int64_t) (w->nb[1] / es),
                                    (int64_t) (w->nb[2] / es), (int) w->ne[0], (int) w->ne[1], (int) w->ne[2], *scratch, s);
    if (e != hipSuccess) return hip_fail(e, "conv kernel pack");
    *rows = *scratch;
    *ld = w->ne[0] * w->ne[1];
    *scratch += conv_pack_bytes(w);
    return TSK_OK;
}

// BF16 convolutions with IC % 32 == 0 and OC % 16 == 0 run the cooperative
// tiles of gemm_ks.hip on bf16 input rows (f32 inputs are rounded to bf16
// first -- the conversion ggml_mul_mat applies to its src1 -- into
// B * IW * IC bf16 of scratch); others the grouped GEMM of gemm_group.hip
bool conv_coop(int wtype, int IC, int OC) { return wtype == TSK_TYPE_BF16 && IC % 32 == 0 && OC % 16 == 0; }
size_t conv_cast_bytes(int wtype, int x_f32, int64_t IC, int64_t IW, int64_t B, int64_t OC) {
    return conv_coop(wtype, (int) IC, (int) OC) && x_f32 ? align256((size_t) (B * IW * IC) * 2) : 0;
}

// one convolution GEMM (validated operands): x rows [B][IW][IC] (ld_x, batch
// stride xb in elements), y rows [B * OW][OC] (ld_y); kw-major weight rows.
// swiglu: w3 rows given -> y = silu(x * w) * (x * w3) (BF16 kernels only).
// xcast: conv_cast_bytes() of scratch, or nullptr when that is 0.
int conv_gemm(int wtype, const void *wrows, const void *w3rows, int64_t ld_w, const float *bias, int KW, int IC, int OC,
              const void *x, int x_f32, int64_t ld_x, int64_t xb, int IW, int B, int s0, int p0, int d0, void *y,
              int y_bf16, int64_t ld_y, uint16_t *xcast, hipStream_t s) {
    const int OW = (int) conv_out_len(IW, KW, s0, p0, d0);
    const bool coop = conv_coop(wtype, IC, OC) && (!x_f32 || xcast) && ld_w % 8 == 0 &&
                      ((uintptr_t) wrows & 15) == 0 && ((uintptr_t) w3rows & 15) == 0;
    if (coop && x_f32) {
        hipError_t e = launch_cast_rows_bf16((const float *) x, ld_x, xb, IW, (int64_t) B * IW, IC, xcast, s);
        if (e != hipSuccess) return hip_fail(e, "conv input cast");
        x = xcast;
        x_f32 = 0;
        ld_x = IC;
        xb = (int64_t) IW * IC;
    }
    GemmProblem q;
    memset(&q, 0, sizeof(q));
    q.x = x; q.bias = bias; q.y = y;
    q.ld_x = ld_x; q.ld_w = ld_w; q.ld_y = ld_y;
    q.x_group_stride = xb;
    q.M = OC; q.N = B * OW; q.K = KW * IC; q.splits = 1;
    q.conv_ic = IC; q.conv_iw = IW; q.conv_ow = OW; q.conv_s = s0; q.conv_p = p0; q.conv_d = d0;
    hipError_t e;
    if (wtype == TSK_TYPE_F32) {
        if (w3rows) return fail(TSK_ERR_UNSUPPORTED, "fused SwiGLU needs BF16 kernels");
        q.wf = (const float *) wrows;
        e = launch_gemm_f32(q, y_bf16, s);
    } else {
        GemmGroup g;
        memset(&g, 0, sizeof(g));
        g.nprob = 1;
        q.w = (const uint16_t *) wrows;
        q.w3 = (const uint16_t *) w3rows;
        g.p[0] = q;
        const int epi = w3rows ? (y_bf16 ? EPI_SWIGLU_BF16 : EPI_SWIGLU_F32) : (y_bf16 ? EPI_STORE_BF16 : EPI_STORE_F32);
        e = coop ? launch_gemm_coop(g, epi, s) : launch_gemm_group(g, x_f32 ? GEMM_X_F32 : 0, epi, s);
    }
    return e == hipSuccess ? TSK_OK : hip_fail(e, "conv GEMM launch");
}

// scratch of tsk_conv1d: the kw-major kernel copy and the bf16 input rows
size_t conv1d_ws_bytes(const tsk_tensor *w, const tsk_tensor *x) {
    return conv_pack_bytes(w) + conv_cast_bytes(w->type, x->type == TSK_TYPE_F32, w->ne[1], x->ne[1], x->ne[2], w->ne[2]);
}

int validate_im2col(const tsk_tensor *kernel, const tsk_tensor *x, int s0, int p0, int d0, const tsk_tensor *dst) {
    int rc;
    if (!kernel) return fail(TSK_ERR_INVALID_ARG, "kernel is NULL");
    for (int i = 0; i < 2; ++i)
        if (kernel->ne[i] < 1) return fail(TSK_ERR_SHAPE, "kernel->ne[%d] < 1", i);
    if ((rc = check_tensor(x, "x")) || (rc = check_tensor(dst, "dst"))) return rc;
    if (x->type != TSK_TYPE_F32) return fail(TSK_ERR_TYPE, "x must be F32");
    if (dst->type != TSK_TYPE_F32 && dst->type != TSK_TYPE_F16 && dst->type != TSK_TYPE_BF16)
        return fail(TSK_ERR_TYPE, "dst must be F32, F16 or BF16");
    const int64_t KW = kernel->ne[0], IC = kernel->ne[1];
    if (x->ne[1] != IC || x->ne[3] != 1) return fail(TSK_ERR_SHAPE, "x must be [IW, IC=%lld, N, 1]", (long long) IC);
    if (s0 < 1 || d0 < 1 || p0 < 0) return fail(TSK_ERR_INVALID_ARG, "stride %d, padding %d, dilation %d", s0, p0, d0);
    const int64_t OW = conv_out_len(x->ne[0], KW, s0, p0, d0);
    if (OW < 1) return fail(TSK_ERR_SHAPE, "output length %lld < 1", (long long) OW);
    if (dst->ne[0] != IC * KW || dst->ne[1] != OW || dst->ne[2] != x->ne[2] || dst->ne[3] != 1)
        return fail(TSK_ERR_SHAPE, "dst must be [IC*KW=%lld, OW=%lld, N=%lld, 1]", (long long) (IC * KW), (long long) OW,
                    (long long) x->ne[2]);
    for (int i = 0; i < 3; ++i)
        if (x->nb[i] % 4) return fail(TSK_ERR_STRIDE, "x->nb[%d] not a multiple of 4", i);
    if (!aligned(x->data, 4)) return fail(TSK_ERR_ALIGN, "x data alignment");
    const size_t es = (size_t) elt_size(dst->type);
    if (dst->nb[0] != es) return fail(TSK_ERR_STRIDE, "dst rows must be contiguous");
    if (!rows_uniform(dst) || dst->nb[1] % es) return fail(TSK_ERR_STRIDE, "dst rows must be uniformly strided");
    if (!aligned(dst->data, es)) return fail(TSK_ERR_ALIGN, "dst data alignment");
    return TSK_OK;
}

}  // namespace

extern "C" int tsk_im2col_1d(const tsk_tensor *kernel, const tsk_tensor *x, int s0, int p0, int d0, tsk_tensor *dst,
                             tsk_stream stream) {
    int rc = validate_im2col(kernel, x, s0, p0, d0, dst);
    if (rc) return rc;
    if ((rc = require_init())) return rc;
    const int es = elt_size(dst->type);
    const int et = dst->type;   // the kernel's element codes are the ggml type ids
    const int64_t OW = dst->ne[1];
    hipError_t e = launch_im2col_1d((const float *) x->data, (int64_t) (x->nb[0] / 4), (int64_t) (x->nb[1] / 4),
                                    (int64_t) (x->nb[2] / 4), (int) x->ne[0], (int) x->ne[1], (int) kernel->ne[0],
                                    (int) OW, (int) x->ne[2], s0, p0, d0, dst->data, et, (int64_t) (dst->nb[1] / es),
                                    (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "im2col launch");
}

extern "C" int tsk_conv1d_pack_weight(const tsk_tensor *w, tsk_tensor *dst, tsk_stream stream) {
    int rc;
    if ((rc = check_conv_weight(w, "w")) || (rc = check_conv_weight(dst, "dst"))) return rc;
    if (!same_shape(w, dst) || dst->type != w->type) return fail(TSK_ERR_SHAPE, "dst must have w's shape and type");
    const size_t es = (size_t) elt_size(w->type);
    const int64_t KW = w->ne[0], IC = w->ne[1];
    if ((KW > 1 && dst->nb[0] != (size_t) IC * es) || (IC > 1 && dst->nb[1] != es) ||
        (w->ne[2] > 1 && dst->nb[2] != (size_t) (KW * IC) * es))
        return fail(TSK_ERR_STRIDE, "dst must be kw-major: nb = [IC*es, es, KW*IC*es]");
    if (!aligned(dst->data, 16)) return fail(TSK_ERR_ALIGN, "dst data must be 16-byte aligned");
    if ((rc = require_init())) return rc;
    hipError_t e = launch_conv_pack(w->data, (int) es, (int64_t) (w->nb[0] / es), (int64_t) (w->nb[1] / es),
                                    (int64_t) (w->nb[2] / es), (int) KW, (int) IC, (int) w->ne[2], dst->data,
                                    (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "conv kernel pack");
}

extern "C" int tsk_conv1d(const tsk_tensor *w, const tsk_tensor *bias, const tsk_tensor *x, int s0, int p0, int d0,
                          tsk_tensor *dst, tsk_stream stream) {
    int rc = validate_conv(w, bias, x, s0, p0, d0, dst);
    if (rc) return rc;
    if ((rc = require_init())) return rc;
    hipStream_t s = (hipStream_t) stream;
    char *ws = nullptr;
    const int x_f32 = x->type == TSK_TYPE_F32;
    const size_t cast = conv_cast_bytes(w->type, x_f32, w->ne[1], x->ne[1], x->ne[2], w->ne[2]);
    if ((rc = workspace(s, conv1d_ws_bytes(w, x), (void **) &ws))) return rc;
    uint16_t *xcast = cast ? (uint16_t *) ws : nullptr;
    char *pk = ws + cast;
    const void *wr = nullptr;
    int64_t ld_w = 0;
    if ((rc = conv_weight_rows(w, &pk, &wr, &ld_w, s))) return rc;
    const int esx = elt_size(x->type), esy = elt_size(dst->type);
    return conv_gemm(w->type, wr, nullptr, ld_w, bias ? (const float *) bias->data : nullptr, (int) w->ne[0],
                     (int) w->ne[1], (int) w->ne[2], x->data, x_f32, (int64_t) (x->nb[1] / esx),
                     (int64_t) (x->nb[2] / esx), (int) x->ne[1], (int) x->ne[2], s0, p0, d0, dst->data,
                     dst->type == TSK_TYPE_BF16, (int64_t) (dst->nb[1] / esy), xcast, s);
}

extern "C" int tsk_swiglu(const tsk_tensor *a, const tsk_tensor *b, tsk_tensor *dst, tsk_stream stream) {
    int rc;
    if ((rc = check_tensor(a, "a")) || (rc = check_tensor(b, "b")) || (rc = check_tensor(dst, "dst"))) return rc;
    if (a->type != TSK_TYPE_F32 || b->type != TSK_TYPE_F32 || dst->type != TSK_TYPE_F32)
        return fail(TSK_ERR_TYPE, "a, b and dst must be F32");
    if (!same_shape(a, b) || !same_shape(a, dst)) return fail(TSK_ERR_SHAPE, "a, b and dst shapes differ");
    if (!contiguous(a) || !contiguous(b) || !contiguous(dst)) return fail(TSK_ERR_STRIDE, "a, b and dst must be contiguous");
    if ((rc = require_init())) return rc;
    const int64_t n = a->ne[0] * a->ne[1] * a->ne[2] * a->ne[3];
    hipError_t e = launch_silu_mul((const float *) a->data, (const float *) b->data, (float *) dst->data, n,
                                   (hipStream_t) stream);
    return e == hipSuccess ? TSK_OK : hip_fail(e, "swiglu launch");
}

namespace {

// scratch of convmlp / mlp: the hidden state [B * OW1][HID] (bf16 for BF16
// kernels: the conversion w2's mul_mat applies), f32 h3 for F32 kernels, the
// bf16 input rows and the kw-major kernel copies
size_t swiglu_mlp_ws_bytes(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2, int KW1, int IC, int HID,
                           int pad, int x_f32, int IW, int B) {
    const int OW1 = (int) conv_out_len(IW, KW1, 1, pad, 1);
    if (OW1 < 1) return 0;
    const bool bf16 = w1->type == TSK_TYPE_BF16;
    const size_t nh = (size_t) B * OW1 * HID;
    const size_t hbytes = align256(nh * (bf16 ? 2 : 4)), h3bytes = bf16 ? 0 : align256(nh * 4);
    return hbytes + h3bytes + conv_cast_bytes(w1->type, x_f32, IC, IW, B, HID) + conv_pack_bytes(w1) +
           conv_pack_bytes(w3) + conv_pack_bytes(w2);
}

// convmlp / mlp on validated operands: geometry of the two convolutions
// (KW = 1, p = 0 for mlp), x rows [B][IW][IC], dst rows [B * OW2][OC]
int swiglu_mlp(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2, int KW1, int IC, int HID, int KW2,
               int OC, int pad, const void *x, int x_f32, int64_t ld_x, int64_t xb, int IW, int B, void *y, int y_bf16,
               int64_t ld_y, hipStream_t s) {
    const int OW1 = (int) conv_out_len(IW, KW1, 1, pad, 1);
    const int OW2 = (int) conv_out_len(OW1, KW2, 1, pad, 1);
    if (OW1 < 1 || OW2 < 1) return fail(TSK_ERR_SHAPE, "output length < 1");
    const bool bf16 = w1->type == TSK_TYPE_BF16;
    const size_t nh = (size_t) B * OW1 * HID;
    const size_t hbytes = align256(nh * (bf16 ? 2 : 4)), h3bytes = bf16 ? 0 : align256(nh * 4);
    const size_t cast = conv_cast_bytes(w1->type, x_f32, IC, IW, B, HID);
    char *ws = nullptr;
    int rc;
    if ((rc = workspace(s, swiglu_mlp_ws_bytes(w1, w3, w2, KW1, IC, HID, pad, x_f32, IW, B), (void **) &ws))) return rc;
    void *h = ws;
    float *h3 = bf16 ? nullptr : (float *) (ws + hbytes);
    uint16_t *xcast = cast ? (uint16_t *) (ws + hbytes + h3bytes) : nullptr;
    char *pk = ws + hbytes + h3bytes + cast;
    const void *r1, *r3, *r2;
    int64_t ld1, ld3, ld2;
    if ((rc = conv_weight_rows(w1, &pk, &r1, &ld1, s)) || (rc = conv_weight_rows(w3, &pk, &r3, &ld3, s)) ||
        (rc = conv_weight_rows(w2, &pk, &r2, &ld2, s)))
        return rc;
    if (ld1 != ld3) return fail(TSK_ERR_STRIDE, "w1 and w3 row strides differ");
    if (bf16) {
        if ((rc = conv_gemm(TSK_TYPE_BF16, r1, r3, ld1, nullptr, KW1, IC, HID, x, x_f32, ld_x, xb, IW, B, 1, pad, 1, h,
                            1, HID, xcast, s)))
            return rc;
    } else {
        if ((rc = conv_gemm(TSK_TYPE_F32, r1, nullptr, ld1, nullptr, KW1, IC, HID, x, 1, ld_x, xb, IW, B, 1, pad, 1, h,
                            0, HID, nullptr, s)) ||
            (rc = conv_gemm(TSK_TYPE_F32, r3, nullptr, ld3, nullptr, KW1, IC, HID, x, 1, ld_x, xb, IW, B, 1, pad, 1, h3,
                            0, HID, nullptr, s)))
            return rc;
        hipError_t e = launch_silu_mul((const float *) h, h3, (float *) h, (int64_t) nh, s);
        if (e != hipSuccess) return hip_fail(e, "swiglu launch");
    }
    return conv_gemm(w2->type, r2, nullptr, ld2, nullptr, KW2, HID, OC, h, !bf16, HID, (int64_t) OW1 * HID, OW1, B, 1,
                     pad, 1, y, y_bf16, ld_y, nullptr, s);
}

int check_mlp_types(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2, const tsk_tensor *x) {
    if (w1->type != w3->type || w1->type != w2->type) return fail(TSK_ERR_TYPE, "w1, w3 and w2 must share one type");
    if (w1->type == TSK_TYPE_F32 && x->type != TSK_TYPE_F32) return fail(TSK_ERR_TYPE, "F32 kernels need F32 x");
    return TSK_OK;
}

}  // namespace

namespace {

int validate_conv_mlp(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2, const tsk_tensor *x,
                      const tsk_tensor *dst) {
    int rc;
    if ((rc = check_conv_weight(w1, "w1")) || (rc = check_conv_weight(w3, "w3")) || (rc = check_conv_weight(w2, "w2")) ||
        (rc = check_conv_act(x, "x")) || (rc = check_conv_act(dst, "dst")))
        return rc;
    if ((rc = check_mlp_types(w1, w3, w2, x))) return rc;
    if (!same_shape(w1, w3)) return fail(TSK_ERR_SHAPE, "w1 and w3 shapes differ");
    const int64_t KW1 = w1->ne[0], IC = w1->ne[1], HID = w1->ne[2], KW2 = w2->ne[0], OC = w2->ne[2];
    if (x->ne[0] != IC) return fail(TSK_ERR_SHAPE, "x->ne[0] != IC=%lld", (long long) IC);
    if (w2->ne[1] != HID) return fail(TSK_ERR_SHAPE, "w2 must be [KW, HID=%lld, OC]", (long long) HID);
    if (IC % 8 || HID % 8) return fail(TSK_ERR_SHAPE, "IC and HID must be multiples of 8");
    const int64_t OW1 = conv_out_len(x->ne[1], KW1, 1, 1, 1), OW2 = conv_out_len(OW1, KW2, 1, 1, 1);
    if (OW1 < 1 || OW2 < 1) return fail(TSK_ERR_SHAPE, "output length < 1");
    if (dst->ne[0] != OC || dst->ne[1] != OW2 || dst->ne[2] != x->ne[2])
        return fail(TSK_ERR_SHAPE, "dst must be [OC=%lld, OW=%lld, B=%lld, 1]", (long long) OC, (long long) OW2,
                    (long long) x->ne[2]);
    if (!rows_uniform(dst)) return fail(TSK_ERR_STRIDE, "dst rows must be uniformly strided");
    if (KW1 * IC > (1 << 30) || KW2 * HID > (1 << 30) || OW1 * x->ne[2] * HID > ((int64_t) 1 << 40))
        return fail(TSK_ERR_SHAPE, "convmlp too large");
    return TSK_OK;
}

}  // namespace

extern "C" int tsk_conv_mlp_swiglu(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2,
                                   const tsk_tensor *x, tsk_tensor *dst, tsk_stream stream) {
    int rc = validate_conv_mlp(w1, w3, w2, x, dst);
    if (rc) return rc;
    const int64_t KW1 = w1->ne[0], IC = w1->ne[1], HID = w1->ne[2], KW2 = w2->ne[0], OC = w2->ne[2];
    if ((rc = require_init())) return rc;
    const int esx = elt_size(x->type), esy = elt_size(dst->type);
    return swiglu_mlp(w1, w3, w2, (int) KW1, (int) IC, (int) HID, (int) KW2, (int) OC, 1, x->data,
                      x->type == TSK_TYPE_F32, (int64_t) (x->nb[1] / esx), (int64_t) (x->nb[2] / esx), (int) x->ne[1],
                      (int) x->ne[2], dst->data, dst->type == TSK_TYPE_BF16, (int64_t) (dst->nb[1] / esy),
                      (hipStream_t) stream);
}

namespace {

// a linear weight [K, M] (rows contiguous) as the kw-major conv kernel [1, K, M]
tsk_tensor linear_as_kernel(const tsk_tensor *w) {
    const size_t es = (size_t) elt_size(w->type);
    tsk_tensor k;
    k.type = w->type;
    k.ne[0] = 1; k.ne[1] = w->ne[0]; k.ne[2] = w->ne[1]; k.ne[3] = 1;
    k.nb[0] = (size_t) w->ne[0] * es; k.nb[1] = es; k.nb[2] = w->nb[1]; k.nb[3] = w->nb[1] * (size_t) w->ne[1];
    k.data = w->data;
    return k;
}

int validate_mlp(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2, const tsk_tensor *x,
                 const tsk_tensor *dst) {
    int rc;
    if ((rc = check_tensor(w1, "w1")) || (rc = check_tensor(w3, "w3")) || (rc = check_tensor(w2, "w2")) ||
        (rc = check_tensor(x, "x")) || (rc = check_tensor(dst, "dst")))
        return rc;
    if ((rc = check_mlp_types(w1, w3, w2, x))) return rc;
    for (const tsk_tensor *w : {w1, w3, w2}) {
        if (w->type != TSK_TYPE_BF16 && w->type != TSK_TYPE_F32) return fail(TSK_ERR_TYPE, "weights must be BF16 or F32");
        if (w->ne[2] != 1 || w->ne[3] != 1) return fail(TSK_ERR_SHAPE, "weights must be 2-D");
        if ((rc = check_rows(w, "w", 16))) return rc;
    }
    if (!same_shape(w1, w3)) return fail(TSK_ERR_SHAPE, "w1 and w3 shapes differ");
    const int64_t IC = w1->ne[0], HID = w1->ne[1], OC = w2->ne[1];
    if (w2->ne[0] != HID) return fail(TSK_ERR_SHAPE, "w2 must be [HID=%lld, OC]", (long long) HID);
    if (x->ne[0] != IC) return fail(TSK_ERR_SHAPE, "x->ne[0] != IC=%lld", (long long) IC);
    if (IC % 8 || HID % 8) return fail(TSK_ERR_SHAPE, "IC and HID must be multiples of 8");
    if (x->type != TSK_TYPE_F32 && x->type != TSK_TYPE_BF16) return fail(TSK_ERR_TYPE, "x must be F32 or BF16");
    if (dst->type != TSK_TYPE_F32 && dst->type != TSK_TYPE_BF16) return fail(TSK_ERR_TYPE, "dst must be F32 or BF16");
    if (dst->ne[0] != OC || dst->ne[1] != x->ne[1] || dst->ne[2] != x->ne[2] || dst->ne[3] != x->ne[3])
        return fail(TSK_ERR_SHAPE, "dst must be [OC=%lld, N, n2, n3] of x", (long long) OC);
    if ((rc = check_rows(x, "x", 16)) || (rc = check_rows(dst, "dst", 16))) return rc;
    if (!rows_uniform(x) || !rows_uniform(dst)) return fail(TSK_ERR_STRIDE, "x and dst rows must be uniformly strided");
    const int64_t N = x->ne[1] * x->ne[2] * x->ne[3];
    if (N > (1 << 30)) return fail(TSK_ERR_SHAPE, "too many rows");
    return TSK_OK;
}

}  // namespace

extern "C" int tsk_mlp_swiglu(const tsk_tensor *w1, const tsk_tensor *w3, const tsk_tensor *w2, const tsk_tensor *x,
                              tsk_tensor *dst, tsk_stream stream) {
    int rc = validate_mlp(w1, w3, w2, x, dst);
    if (rc) return rc;
    const int64_t IC = w1->ne[0], HID = w1->ne[1], OC = w2->ne[1];
    const int64_t N = x->ne[1] * x->ne[2] * x->ne[3];
    if ((rc = require_init())) return rc;
    // a linear layer is the KW = 1, padding 0 convolution over one sequence of N rows
    const int esx = elt_size(x->type), esy = elt_size(dst->type);
    const tsk_tensor k1 = linear_as_kernel(w1), k3 = linear_as_kernel(w3), k2 = linear_as_kernel(w2);
    return swiglu_mlp(&k1, &k3, &k2, 1, (int) IC, (int) HID, 1, (int) OC, 0, x->data, x->type == TSK_TYPE_F32,
                      (int64_t) (x->nb[1] / esx), 0, (int) N, 1, dst->data, dst->type == TSK_TYPE_BF16,
                      (int64_t) (dst->nb[1] / esy), (hipStream_t) stream);
}

// ------------------------------------------------------------------ supports_op
extern "C" int tsk_supports_op(int op, const tsk_tensor *const *srcs, int n_srcs, const tsk_tensor *dst) {
    // validation only: swap data pointers for a dummy aligned address
    static char dummy[64] __attribute__((aligned(64)));
    tsk_tensor t[6], d;
    if (!srcs || !dst || n_srcs < 1 || n_srcs > 5) return 0;
    for (int i = 0; i < n_srcs; ++i) {
        if (!srcs[i]) { t[i].type = -1; continue; }
        t[i] = *srcs[i];
        t[i].data = dummy;
    }
    d = *dst;
    d.data = dummy;
    auto opt = [&](int i) -> const tsk_tensor * { return i < n_srcs && srcs[i] ? &t[i] : nullptr; };
    int rc;
    switch (op) {
        case TSK_OP_MUL_MAT:
            rc = n_srcs >= 2 ? validate_mul_mat(&t[0], &t[1], opt(2), &d) : TSK_ERR_INVALID_ARG;
            break;
        case TSK_OP_FLASH_ATTN_EXT:
            rc = n_srcs >= 3 ? validate_fa(&t[0], &t[1], &t[2], opt(3), 0.125f, 0.0f, 0.0f, TSK_PREC_F32, &d)
                             : TSK_ERR_INVALID_ARG;
            break;
        case TSK_OP_RMS_NORM_MUL:
            rc = check_unary(&t[0], &d);
            if (!rc && opt(1)) rc = check_w(&t[1], t[0].ne[0]);
            break;
        case TSK_OP_ROPE_EXT:
            rc = check_unary(&t[0], &d);
            if (!rc) rc = n_srcs >= 2 ? check_pos(&t[1], &t[0]) : TSK_ERR_INVALID_ARG;
            break;
        case TSK_OP_NORM:
            rc = check_unary(&t[0], &d);
            break;
        case TSK_OP_IM2COL:
            rc = n_srcs >= 2 ? validate_im2col(&t[0], &t[1], 1, 1, 1, &d) : TSK_ERR_INVALID_ARG;
            break;
        case TSK_OP_CONV1D:
            rc = n_srcs >= 2 ? validate_conv(&t[0], opt(2), &t[1], 1, 1, 1, &d) : TSK_ERR_INVALID_ARG;
            break;
        default:
            rc = TSK_ERR_UNSUPPORTED;
    }
    return rc == TSK_OK ? 1 : 0;
}

// ------------------------------------------------------------------ workspace_size
extern "C" int tsk_workspace_size(int op, const tsk_tensor *const *srcs, int n_srcs, const tsk_tensor *dst,
                                  size_t *bytes) {
    // validation only: data pointers are swapped for a dummy aligned address
    static char dummy[64] __attribute__((aligned(64)));
    if (!bytes) return fail(TSK_ERR_INVALID_ARG, "bytes is NULL");
    *bytes = 0;
    if (!srcs || !dst || n_srcs < 1 || n_srcs > 5) return fail(TSK_ERR_INVALID_ARG, "srcs / dst");
    tsk_tensor t[5], d = *dst;
    for (int i = 0; i < n_srcs; ++i) {
        if (!srcs[i]) { t[i].type = -1; continue; }
        t[i] = *srcs[i];
        t[i].data = dummy;
    }
    d.data = dummy;
    auto opt = [&](int i) -> const tsk_tensor * { return i < n_srcs && srcs[i] ? &t[i] : nullptr; };
    auto need = [&](int n) { return n_srcs >= n ? TSK_OK : fail(TSK_ERR_INVALID_ARG, "op %d needs %d srcs", op, n); };
    int rc;
    switch (op) {
        case TSK_OP_MUL_MAT:
            if ((rc = need(2)) || (rc = validate_mul_mat(&t[0], &t[1], opt(2), &d))) return rc;
            *bytes = plan_mul_mat(&t[0], &t[1], &d).bytes;
            return TSK_OK;
        case TSK_OP_FLASH_ATTN_EXT:
            if ((rc = need(3)) || (rc = validate_fa(&t[0], &t[1], &t[2], opt(3), 0.125f, 0.0f, 0.0f, TSK_PREC_F32, &d)))
                return rc;
            *bytes = fa_ws_bytes(&t[0], &t[1], &t[2], opt(3), 0.0f, 0.0f, &d);
            return TSK_OK;
        case TSK_OP_CONV1D:
            if ((rc = need(2)) || (rc = validate_conv(&t[0], opt(2), &t[1], 1, 1, 1, &d))) return rc;
            *bytes = conv1d_ws_bytes(&t[0], &t[1]);
            return TSK_OK;
        case TSK_OP_CONV_MLP_SWIGLU:
            if ((rc = need(4)) || (rc = validate_conv_mlp(&t[0], &t[1], &t[2], &t[3], &d))) return rc;
            *bytes = swiglu_mlp_ws_bytes(&t[0], &t[1], &t[2], (int) t[0].ne[0], (int) t[0].ne[1], (int) t[0].ne[2], 1,
                                         t[3].type == TSK_TYPE_F32, (int) t[3].ne[1], (int) t[3].ne[2]);
            return TSK_OK;
        case TSK_OP_MLP_SWIGLU:
            if ((rc = need(4)) || (rc = validate_mlp(&t[0], &t[1], &t[2], &t[3], &d))) return rc;
        {
            // linear layers are k = 1, padding 0 convolutions over the N rows
            const tsk_tensor k1 = linear_as_kernel(&t[0]), k3 = linear_as_kernel(&t[1]), k2 = linear_as_kernel(&t[2]);
            *bytes = swiglu_mlp_ws_bytes(&k1, &k3, &k2, 1, (int) t[0].ne[0], (int) t[0].ne[1], 0,
                                         t[3].type == TSK_TYPE_F32, (int) (t[3].ne[1] * t[3].ne[2] * t[3].ne[3]), 1);
            return TSK_OK;
        }
        case TSK_OP_RMS_NORM_Q8_0:
            if ((rc = need(2)) || (rc = validate_rms_norm_q8(&t[0], &t[1], &d))) return rc;
            *bytes = rms_norm_q8_ws_bytes(&t[0]);
            return TSK_OK;
        case TSK_OP_RMS_NORM_MUL: case TSK_OP_ROPE_EXT: case TSK_OP_NORM: case TSK_OP_IM2COL:
            return TSK_OK;   // no scratch
        default:
            return fail(TSK_ERR_UNSUPPORTED, "op %d", op);
    }
}
