// gguf.cpp — GGUF ingestion (the reference's on-disk model format, read by
// ts_model::load_backend, src/common/ts_model.cpp:13-41, through ggml's
// gguf_init_from_file): a reader of GGUF v2/v3 headers, metadata and tensor
// tables, tensor reads as stored or converted to f32, and the loaders that
// hand the converter's tensors (convert/convert_thinksound.py:32,
// convert/quantize_gguf.py:9-45) to the DiT and T5 drivers by name.
//
// Layout read (GGUF v3, little endian): magic "GGUF", u32 version, u64
// tensor count, u64 metadata count; metadata = (string key, u32 type,
// value); tensor infos = (string name, u32 n_dims, u64 ne[n_dims], u32 ggml
// type, u64 offset); tensor data from the first multiple of
// general.alignment (default 32) after the infos, each tensor at its offset.
// Strings are u64 length + bytes. Host-only code: no HIP call here except
// through the drivers' set_tensor entry points.
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/tsk/tsk.h"
#include "tsk_runtime.h"

using namespace tsk;

namespace {

enum GType : uint32_t {
    GT_U8 = 0, GT_I8 = 1, GT_U16 = 2, GT_I16 = 3, GT_U32 = 4, GT_I32 = 5, GT_F32 = 6, GT_BOOL = 7,
    GT_STRING = 8, GT_ARRAY = 9, GT_U64 = 10, GT_I64 = 11, GT_F64 = 12
};

struct KV {
    uint32_t type;
    uint64_t u;          // integer / bool value
    double f;            // float value
    std::string s;
};

struct TInfo {
    std::string name;
    int64_t ne[4];
    uint32_t type;
    uint64_t offset;
};

size_t scalar_size(uint32_t t) {
    switch (t) {
        case GT_U8: case GT_I8: case GT_BOOL: return 1;
        case GT_U16: case GT_I16: return 2;
        case GT_U32: case GT_I32: case GT_F32: return 4;
        case GT_U64: case GT_I64: case GT_F64: return 8;
        default: return 0;
    }
}

// bytes of a tensor of ggml type `type` with ne (0 if the type is not supported)
uint64_t tensor_bytes(uint32_t type, const int64_t ne[4]) {
    const uint64_t rows = (uint64_t) ne[1] * ne[2] * ne[3];
    switch (type) {
        case TSK_TYPE_F32: return 4ull * ne[0] * rows;
        case TSK_TYPE_F16: case TSK_TYPE_BF16: return 2ull * ne[0] * rows;
        case TSK_TYPE_Q8_0: return ne[0] % 32 ? 0 : 34ull * (ne[0] / 32) * rows;
        default: return 0;
    }
}

float half_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t) (h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t u;
    if (e == 0) {
        if (m == 0) u = s;
        else {   // subnormal: m * 2^-24, exact in f32
            float f = (float) m * (1.0f / 16777216.0f);
            memcpy(&u, &f, 4);
            u |= s;
        }
    } else if (e == 31) {
        u = s | 0x7f800000u | (m << 13);
    } else {
        u = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

}  // namespace

struct tsk_gguf {
    FILE *f = nullptr;
    uint32_t version = 0;
    uint64_t data_start = 0, file_size = 0;
    std::unordered_map<std::string, KV> kv;
    std::vector<TInfo> t;
    std::unordered_map<std::string, size_t> tidx;
};

namespace {

struct Rd {
    FILE *f;
    bool ok = true;
    template <class T> T get() {
        T v{};
        if (ok && fread(&v, sizeof(T), 1, f) != 1) ok = false;
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (1u << 20)) { ok = false; return std::string(); }
        std::string s((size_t) n, '\0');
        if (n && fread(&s[0], 1, (size_t) n, f) != n) ok = false;
        return s;
    }
    void skip(uint64_t n) {
        if (ok && fseeko(f, (off_t) n, SEEK_CUR) != 0) ok = false;
    }
};

int parse(tsk_gguf *g) {
    Rd r{g->f};
    const uint32_t magic = r.get<uint32_t>();
    if (!r.ok || magic != 0x46554747u) return fail(TSK_ERR_INVALID_ARG, "not a GGUF file (magic)");
    g->version = r.get<uint32_t>();
    if (g->version < 2 || g->version > 3) return fail(TSK_ERR_UNSUPPORTED, "GGUF version %u", g->version);
    const uint64_t nt = r.get<uint64_t>(), nkv = r.get<uint64_t>();
    if (!r.ok || nt > (1u << 24) || nkv > (1u << 24)) return fail(TSK_ERR_INVALID_ARG, "GGUF header counts");
    for (uint64_t i = 0; i < nkv && r.ok; ++i) {
        const std::string key = r.str();
        KV v;
        v.type = r.get<uint32_t>();
        v.u = 0;
        v.f = 0.0;
        if (v.type == GT_STRING) {
            v.s = r.str();
        } else if (v.type == GT_ARRAY) {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t n = r.get<uint64_t>();
            if (et == GT_STRING) {
                for (uint64_t j = 0; j < n && r.ok; ++j) (void) r.str();
            } else {
                const size_t es = scalar_size(et);
                if (!es) return fail(TSK_ERR_INVALID_ARG, "GGUF array of type %u", et);
                r.skip(n * es);
            }
            v.u = n;
        } else {
            const size_t es = scalar_size(v.type);
            if (!es) return fail(TSK_ERR_INVALID_ARG, "GGUF metadata '%s' of type %u", key.c_str(), v.type);
            unsigned char b[8] = {0};
            if (r.ok && fread(b, es, 1, g->f) != 1) r.ok = false;
            switch (v.type) {
                case GT_F32: { float x; memcpy(&x, b, 4); v.f = x; break; }
                case GT_F64: { double x; memcpy(&x, b, 8); v.f = x; break; }
                case GT_I8: v.u = (uint64_t) (int64_t) (int8_t) b[0]; break;
                case GT_I16: { int16_t x; memcpy(&x, b, 2); v.u = (uint64_t) (int64_t) x; break; }
                case GT_I32: { int32_t x; memcpy(&x, b, 4); v.u = (uint64_t) (int64_t) x; break; }
                default: memcpy(&v.u, b, es); break;
            }
            v.f = v.type == GT_F32 || v.type == GT_F64 ? v.f : (double) (int64_t) v.u;
        }
        g->kv[key] = v;
    }
    for (uint64_t i = 0; i < nt && r.ok; ++i) {
        TInfo ti;
        ti.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (!r.ok || nd < 1 || nd > 4) return fail(TSK_ERR_INVALID_ARG, "GGUF tensor '%s' has %u dims", ti.name.c_str(), nd);
        for (int d = 0; d < 4; ++d) ti.ne[d] = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            const uint64_t n = r.get<uint64_t>();
            if (n == 0 || n > (1ull << 40)) r.ok = false;
            ti.ne[d] = (int64_t) n;
        }
        ti.type = r.get<uint32_t>();
        ti.offset = r.get<uint64_t>();
        if (!r.ok) break;
        g->tidx[ti.name] = g->t.size();
        g->t.push_back(ti);
    }
    if (!r.ok) return fail(TSK_ERR_INVALID_ARG, "GGUF file truncated or malformed");
    uint64_t align = 32;
    auto it = g->kv.find("general.alignment");
    if (it != g->kv.end() && it->second.type == GT_U32 && it->second.u) align = it->second.u;
    const uint64_t pos = (uint64_t) ftello(g->f);
    g->data_start = (pos + align - 1) / align * align;
    if (fseeko(g->f, 0, SEEK_END) != 0) return fail(TSK_ERR_INVALID_ARG, "GGUF seek");
    g->file_size = (uint64_t) ftello(g->f);
    for (const TInfo &ti : g->t) {
        const uint64_t nb = tensor_bytes(ti.type, ti.ne);
        if (nb && g->data_start + ti.offset + nb > g->file_size)
            return fail(TSK_ERR_INVALID_ARG, "GGUF tensor '%s' runs past the end of the file", ti.name.c_str());
    }
    return TSK_OK;
}

const TInfo *find(const tsk_gguf *g, const char *name) {
    auto it = g->tidx.find(name);
    return it == g->tidx.end() ? nullptr : &g->t[it->second];
}

}  // namespace

extern "C" int tsk_gguf_open(const char *path, tsk_gguf **out) {
    if (!path || !out) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    *out = nullptr;
    tsk_gguf *g = new tsk_gguf();
    g->f = fopen(path, "rb");
    if (!g->f) {
        delete g;
        return fail(TSK_ERR_INVALID_ARG, "cannot open '%s'", path);
    }
    const int rc = parse(g);
    if (rc) {
        tsk_gguf_close(g);
        return rc;
    }
    *out = g;
    return TSK_OK;
}

extern "C" void tsk_gguf_close(tsk_gguf *g) {
    if (!g) return;
    if (g->f) fclose(g->f);
    delete g;
}

extern "C" int tsk_gguf_n_tensors(const tsk_gguf *g) { return g ? (int) g->t.size() : 0; }

extern "C" int tsk_gguf_tensor_info(const tsk_gguf *g, int i, const char **name, int64_t ne[4], int *type) {
    if (!g || i < 0 || i >= (int) g->t.size()) return fail(TSK_ERR_INVALID_ARG, "tensor index %d", i);
    if (name) *name = g->t[i].name.c_str();
    if (ne) for (int d = 0; d < 4; ++d) ne[d] = g->t[i].ne[d];
    if (type) *type = (int) g->t[i].type;
    return TSK_OK;
}

extern "C" int tsk_gguf_find_tensor(const tsk_gguf *g, const char *name, int64_t ne[4], int *type) {
    if (!g || !name) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    const TInfo *ti = find(g, name);
    if (!ti) return fail(TSK_ERR_INVALID_ARG, "no tensor '%s' in the GGUF file", name);
    if (ne) for (int d = 0; d < 4; ++d) ne[d] = ti->ne[d];
    if (type) *type = (int) ti->type;
    return (int) (ti - g->t.data());
}

extern "C" int tsk_gguf_read_tensor(const tsk_gguf *g, const char *name, int as_f32, void *dst, size_t dst_bytes) {
    if (!g || !name || !dst) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    const TInfo *ti = find(g, name);
    if (!ti) return fail(TSK_ERR_INVALID_ARG, "no tensor '%s' in the GGUF file", name);
    const uint64_t nb = tensor_bytes(ti->type, ti->ne);
    if (!nb) return fail(TSK_ERR_TYPE, "tensor '%s' has unsupported type %u", name, ti->type);
    const uint64_t n = (uint64_t) ti->ne[0] * ti->ne[1] * ti->ne[2] * ti->ne[3];
    const uint64_t want = as_f32 ? 4 * n : nb;
    if (dst_bytes != want) return fail(TSK_ERR_SHAPE, "tensor '%s' needs %llu bytes, got %zu", name,
                                       (unsigned long long) want, dst_bytes);
    std::vector<unsigned char> raw;
    unsigned char *buf = (unsigned char *) dst;
    if (as_f32 && ti->type != TSK_TYPE_F32) {
        raw.resize((size_t) nb);
        buf = raw.data();
    }
    if (fseeko(g->f, (off_t) (g->data_start + ti->offset), SEEK_SET) != 0 || fread(buf, 1, (size_t) nb, g->f) != nb)
        return fail(TSK_ERR_INVALID_ARG, "read of tensor '%s' failed", name);
    if (!as_f32 || ti->type == TSK_TYPE_F32) return TSK_OK;
    float *o = (float *) dst;
    if (ti->type == TSK_TYPE_F16) {
        for (uint64_t i = 0; i < n; ++i) { uint16_t h; memcpy(&h, raw.data() + 2 * i, 2); o[i] = half_to_f32(h); }
    } else if (ti->type == TSK_TYPE_BF16) {
        for (uint64_t i = 0; i < n; ++i) {
            uint16_t h; memcpy(&h, raw.data() + 2 * i, 2);
            const uint32_t u = (uint32_t) h << 16;
            memcpy(&o[i], &u, 4);
        }
    } else {   // Q8_0: fp32(d) * q, exact
        for (uint64_t b = 0; b < n / 32; ++b) {
            const unsigned char *blk = raw.data() + 34 * b;
            uint16_t dh; memcpy(&dh, blk, 2);
            const float d = half_to_f32(dh);
            for (int j = 0; j < 32; ++j) o[32 * b + j] = d * (float) (int8_t) blk[2 + j];
        }
    }
    return TSK_OK;
}

extern "C" int tsk_gguf_get_u32(const tsk_gguf *g, const char *key, uint32_t *out) {
    if (!g || !key || !out) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(TSK_ERR_INVALID_ARG, "no metadata '%s'", key);
    const KV &v = it->second;
    if (v.type == GT_STRING || v.type == GT_ARRAY || v.type == GT_F32 || v.type == GT_F64)
        return fail(TSK_ERR_TYPE, "metadata '%s' is not an integer", key);
    *out = (uint32_t) v.u;
    return TSK_OK;
}

extern "C" int tsk_gguf_get_f32(const tsk_gguf *g, const char *key, float *out) {
    if (!g || !key || !out) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(TSK_ERR_INVALID_ARG, "no metadata '%s'", key);
    const KV &v = it->second;
    if (v.type == GT_STRING || v.type == GT_ARRAY) return fail(TSK_ERR_TYPE, "metadata '%s' is not a number", key);
    *out = (float) v.f;
    return TSK_OK;
}

extern "C" int tsk_gguf_get_str(const tsk_gguf *g, const char *key, const char **out) {
    if (!g || !key || !out) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(TSK_ERR_INVALID_ARG, "no metadata '%s'", key);
    if (it->second.type != GT_STRING) return fail(TSK_ERR_TYPE, "metadata '%s' is not a string", key);
    *out = it->second.s.c_str();
    return TSK_OK;
}

// ------------------------------------------------------------------ driver loaders
extern "C" int tsk_dit_config_from_gguf(const tsk_gguf *g, tsk_dit_config *c) {
    if (!g || !c) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    // keys of convert/convert_thinksound.py:38-45; absent keys keep the defaults
    auto u = [&](const char *k, int *dst) {
        auto it = g->kv.find(k);
        if (it != g->kv.end() && it->second.type != GT_STRING && it->second.type != GT_ARRAY) *dst = (int) it->second.u;
    };
    auto f = [&](const char *k, float *dst) {
        auto it = g->kv.find(k);
        if (it != g->kv.end() && it->second.type != GT_STRING && it->second.type != GT_ARRAY) *dst = (float) it->second.f;
    };
    u("dit.hidden_dim", &c->hidden);
    u("dit.depth", &c->depth);
    u("dit.fused_depth", &c->fused_depth);
    u("dit.num_heads", &c->n_head);
    u("dit.latent_dim", &c->latent_dim);
    u("dit.text_seq_len", &c->text_seq);
    f("dit.rope_theta", &c->rope_theta);
    f("dit.t_embed_max_period", &c->t_max_period);
    if (c->n_head > 0) c->head_dim = c->hidden / c->n_head;
    return TSK_OK;
}

extern "C" int tsk_t5_config_from_gguf(const tsk_gguf *g, tsk_t5_config *c) {
    if (!g || !c) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    // keys of src/t5_encoder.cpp:31-36
    auto u = [&](const char *k, int *dst) {
        auto it = g->kv.find(k);
        if (it != g->kv.end() && it->second.type != GT_STRING && it->second.type != GT_ARRAY) *dst = (int) it->second.u;
    };
    u("t5.d_model", &c->d_model);
    u("t5.d_ff", &c->d_ff);
    u("t5.n_layers", &c->n_layers);
    u("t5.n_heads", &c->n_heads);
    u("t5.d_kv", &c->d_kv);
    u("t5.rel_buckets", &c->rel_buckets);
    u("t5.rel_max_dist", &c->rel_max_dist);
    auto it = g->kv.find("t5.eps");
    if (it != g->kv.end() && it->second.type != GT_STRING && it->second.type != GT_ARRAY) c->eps = (float) it->second.f;
    return TSK_OK;
}

// every DiT weight by name: Q8_0 tensors the driver stores as Q8_0 bit for
// bit; others converted to f32 on the host (F32 / F16 / BF16 exactly) and
// handed to tsk_dit_set_tensor, which rounds matrices to the driver's BF16 (or
// quantizes the Q8_0 driver's block projections). A Q8_0 tensor the driver
// stores otherwise is refused: bf16(fp32(d) * q) would not run the
// Q8_0 x Q8_0 products the file asks for.
extern "C" int tsk_dit_load_gguf(tsk_dit *dit, const tsk_gguf *g) {
    if (!dit || !g) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    std::vector<float> buf;
    for (int i = 0; i < tsk_dit_n_tensors(dit); ++i) {
        const char *name;
        int64_t ne[4];
        int rc = tsk_dit_tensor_info(dit, i, &name, ne);
        if (rc) return rc;
        const TInfo *ti = find(g, name);
        if (!ti) return fail(TSK_ERR_INVALID_ARG, "GGUF file has no tensor '%s'", name);
        if (ti->ne[0] * ti->ne[1] * ti->ne[2] * ti->ne[3] != ne[0] * ne[1] || ti->ne[0] != ne[0])
            return fail(TSK_ERR_SHAPE, "GGUF tensor '%s' is [%lld, %lld], the driver needs [%lld, %lld]", name,
                        (long long) ti->ne[0], (long long) (ti->ne[1] * ti->ne[2] * ti->ne[3]), (long long) ne[0],
                        (long long) ne[1]);
        const int dtype = tsk_dit_tensor_type(dit, i);
        if (ti->type == TSK_TYPE_Q8_0) {
            if (dtype != TSK_TYPE_Q8_0)
                return fail(TSK_ERR_TYPE, "GGUF tensor '%s' is Q8_0: this DiT driver stores it as type %d", name, dtype);
            std::vector<uint8_t> raw((size_t) (ne[0] / 32) * 34 * (size_t) ne[1]);
            if ((rc = tsk_gguf_read_tensor(g, name, 0, raw.data(), raw.size()))) return rc;
            if ((rc = tsk_dit_set_tensor_q8_0(dit, name, raw.data(), raw.size()))) return rc;
            continue;
        }
        buf.resize((size_t) (ne[0] * ne[1]));
        if ((rc = tsk_gguf_read_tensor(g, name, 1, buf.data(), buf.size() * 4))) return rc;
        if ((rc = tsk_dit_set_tensor(dit, name, buf.data(), (int64_t) buf.size()))) return rc;
    }
    return TSK_OK;
}

// T5 weights in their stored form: Q8_0 blocks for the matrices, F32 vectors
extern "C" int tsk_t5_load_gguf(tsk_t5 *t5, const tsk_gguf *g) {
    if (!t5 || !g) return fail(TSK_ERR_INVALID_ARG, "NULL argument");
    std::vector<unsigned char> buf;
    for (int i = 0; i < tsk_t5_n_tensors(t5); ++i) {
        const char *name;
        int64_t ne[4];
        int type;
        int rc = tsk_t5_tensor_info(t5, i, &name, ne, &type);
        if (rc) return rc;
        const TInfo *ti = find(g, name);
        if (!ti) return fail(TSK_ERR_INVALID_ARG, "GGUF file has no tensor '%s'", name);
        if (ti->ne[0] != ne[0] || ti->ne[1] * ti->ne[2] * ti->ne[3] != ne[1])
            return fail(TSK_ERR_SHAPE, "GGUF tensor '%s' shape differs from the driver's", name);
        if ((int) ti->type != type)
            return fail(TSK_ERR_TYPE, "GGUF tensor '%s' has type %u, the driver needs %d", name, ti->type, type);
        buf.resize((size_t) tensor_bytes(ti->type, ti->ne));
        if ((rc = tsk_gguf_read_tensor(g, name, 0, buf.data(), buf.size()))) return rc;
        if ((rc = tsk_t5_set_tensor(t5, name, buf.data(), buf.size()))) return rc;
    }
    return TSK_OK;
}
