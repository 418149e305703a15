// attn.hip — fused flash attention for gfx950 (ggml_flash_attn_ext semantics,
// the node emitted by attention() in src/mmdit.cpp:85-95).
//
// Work split: one workgroup = NW waves on one (batch, head) and NW*QB*16
// query rows; each wave owns QB blocks of 16 query rows. K/V tiles of 64 keys
// are staged through LDS (double buffered, one barrier per tile) and shared by
// the workgroup's waves.
//
// The kernel computes S^T = K.Q^T (keys x queries) with MFMA so that each lane
// owns ONE query row in the accumulator layout: row max / row sum / rescale
// are lane-local (plus 2 cross-lane steps), and the probabilities P^T come out
// of the S^T accumulators already in the B-operand layout of O^T = V^T.P^T.
// V is therefore staged transposed ([dim][key]) in LDS.
//
// 16-bit K/V: QK^T on bf16 or f16 MFMA (16x16x32), Q converted to K's type as
// ggml-cpu does; P and V enter the P.V MFMA as fp16 (V keeps the F16 cast
// mmdit.cpp:89-90 applies); fp32 logits, softmax and accumulation.
// F32 K/V: fp32 MFMA (16x16x4) throughout.
#include "tsk_common.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

namespace tsk {

namespace {

constexpr int KT = 64;          // keys per LDS tile
constexpr int D = 64;           // head dim
constexpr int LDS16 = D + 8;    // 16-bit row stride (elements): 144 B rows
constexpr int LDS32 = D + 4;    // f32 row stride (elements)

// KS key ranges per workgroup: the waves of range ks take key tiles
// ks, ks + KS, ... for the same NW * QB * 16 query rows (their own LDS
// buffers), and range 0 merges the others' running max / sum / output at the
// end; KS = 2 puts two waves on each SIMD where the grid has one workgroup per CU
template <Elt QE, Elt KVE, Elt OE, int NW, int QB, int KS = 1>
__global__ __launch_bounds__(NW * 64 * KS)
void attn_kernel(const AttnParams p) {
    constexpr bool F32 = (KVE == Elt::F32);
    constexpr int NT = NW * 64;      // threads of one key range
    constexpr int QROWS = NW * QB * 16;

    const int tid = threadIdx.x % NT;
    // wave-uniform: the key range and the wave's query rows stay in scalar registers
    const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x / NT);
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int h = blockIdx.y, b = blockIdx.z;
    const int hk = h / (p.H / p.Hkv);
    const int qbase = blockIdx.x * QROWS + wave * QB * 16;

    const char *qptr = (const char *) p.q + (int64_t) h * p.q_nb2 + (int64_t) b * p.q_nb3;
    const char *kptr = (const char *) p.k + (int64_t) hk * p.k_nb2 + (int64_t) b * p.k_nb3;
    const char *vptr = (const char *) p.v + (int64_t) hk * p.v_nb2 + (int64_t) b * p.v_nb3;

    // ALiBi slope (ggml): 1 unless max_bias > 0
    float slope = 1.0f;
    if (p.max_bias > 0.0f) {
        const uint32_t hh = (uint32_t) h;
        slope = hh < p.n_head_log2 ? __powf(p.m0, (float) (hh + 1))
                                   : __powf(p.m1, (float) (2 * (hh - p.n_head_log2) + 1));
    }

    // ---------------- LDS
    typedef typename std::conditional<F32, float, uint16_t>::type lds_t;
    constexpr int LSTR = F32 ? LDS32 : LDS16;
    __shared__ __attribute__((aligned(16))) lds_t Ks_all[KS][2][KT * LSTR];
    __shared__ __attribute__((aligned(16))) lds_t Vt_all[KS][2][D * LSTR];
    lds_t (*Ks)[KT * LSTR] = Ks_all[ks];
    lds_t (*Vt)[D * LSTR] = Vt_all[ks];

    // ---------------- Q fragments (B operand of S^T = K.Q^T)
    // 16-bit: lane holds Q[q = lr][32*kc + 8*lg + j], j < 8, kc < 2
    // f32   : lane holds Q[q = lr][4*kc + lg], kc < 16
    typedef typename std::conditional<KVE == Elt::BF16, bf16x8, f16x8>::type frag16;
    frag16 qf16[QB][2];
    float qf32[QB][16];
    for (int qb = 0; qb < QB; ++qb) {
        const int qrow = qbase + qb * 16 + lr;
        const bool ok = qrow < p.Nq;
        const char *qr = qptr + (int64_t) (ok ? qrow : 0) * p.q_nb1;
        if constexpr (F32) {
            for (int kc = 0; kc < 16; ++kc)
                qf32[qb][kc] = ok ? load_as_f32<QE>(qr, 4 * kc + lg) : 0.0f;
        } else {
            for (int kc = 0; kc < 2; ++kc) {
                uint16_t tmp[8];
                if constexpr (QE == KVE) {
                    u32x4 raw = ok ? *(const u32x4 *) (qr + (32 * kc + 8 * lg) * 2) : u32x4{0, 0, 0, 0};
                    __builtin_memcpy(tmp, &raw, 16);
                } else {
                    for (int j = 0; j < 8; ++j) {
                        const float x = ok ? load_as_f32<QE>(qr, 32 * kc + 8 * lg + j) : 0.0f;
                        tmp[j] = KVE == Elt::BF16 ? f32_to_bf16_bits(x) : f32_to_f16_bits(x);
                    }
                }
                __builtin_memcpy(&qf16[qb][kc], tmp, 16);
            }
        }
    }

    // ---------------- accumulators
    f32x4 oacc[QB][4];
    float m_run[QB], l_run[QB];
    for (int qb = 0; qb < QB; ++qb) {
        for (int dt = 0; dt < 4; ++dt) oacc[qb][dt] = f32x4{0, 0, 0, 0};
        m_run[qb] = -INFINITY;
        l_run[qb] = 0.0f;
    }

    // ---------------- global -> register staging of one K/V tile
    // 16-bit: K = 512 chunks of 16 B (key, 8 dims); V = 256 pairs of keys x 8 dims
    // f32   : K = 1024 chunks of 16 B (key, 4 dims); V = 512 pairs of keys x 4 dims
    constexpr int KCH = F32 ? 1024 : 512;
    constexpr int VCH = F32 ? 512 : 256;
    constexpr int KPER = (KCH + NT - 1) / NT;
    constexpr int VPER = (VCH + NT - 1) / NT;
    constexpr int CPR = F32 ? 16 : 8;          // 16-B chunks per row
    u32x4 kreg[KPER];
    u32x4 vreg[VPER][2];

    const int ntiles = (p.Nkv + KT - 1) / KT;
    const int niter = (ntiles + KS - 1) / KS;   // the same count in every key range

    auto gload = [&](int tile) {
        const int k0 = tile * KT;
        for (int i = 0; i < KPER; ++i) {
            const int c = tid + i * NT;
            kreg[i] = u32x4{0, 0, 0, 0};
            if (c < KCH) {
                const int key = k0 + c / CPR, ch = c % CPR;
                if (key < p.Nkv) kreg[i] = *(const u32x4 *) (kptr + (int64_t) key * p.k_nb1 + ch * 16);
            }
        }
        for (int i = 0; i < VPER; ++i) {
            const int c = tid + i * NT;
            vreg[i][0] = vreg[i][1] = u32x4{0, 0, 0, 0};
            if (c < VCH) {
                const int key = k0 + 2 * (c / CPR), ch = c % CPR;
                if (key < p.Nkv) vreg[i][0] = *(const u32x4 *) (vptr + (int64_t) key * p.v_nb1 + ch * 16);
                if (key + 1 < p.Nkv) vreg[i][1] = *(const u32x4 *) (vptr + (int64_t) (key + 1) * p.v_nb1 + ch * 16);
            }
        }
    };
    auto lstore = [&](int buf) {
        for (int i = 0; i < KPER; ++i) {
            const int c = tid + i * NT;
            if (c < KCH) {
                const int key = c / CPR, ch = c % CPR;
                *(u32x4 *) &Ks[buf][key * LSTR + ch * (16 / sizeof(lds_t))] = kreg[i];
            }
        }
        for (int i = 0; i < VPER; ++i) {
            const int c = tid + i * NT;
            if (c < VCH) {
                const int kp = 2 * (c / CPR), ch = c % CPR;
                if constexpr (F32) {
                    const float *v0 = (const float *) &vreg[i][0];
                    const float *v1 = (const float *) &vreg[i][1];
                    for (int j = 0; j < 4; ++j) {
                        const int d = ch * 4 + j;
                        Vt[buf][d * LSTR + kp] = v0[j];
                        Vt[buf][d * LSTR + kp + 1] = v1[j];
                    }
                } else {
                    const uint16_t *v0 = (const uint16_t *) &vreg[i][0];
                    const uint16_t *v1 = (const uint16_t *) &vreg[i][1];
                    for (int j = 0; j < 8; ++j) {
                        uint16_t a0 = v0[j], a1 = v1[j];
                        if constexpr (KVE == Elt::BF16) {   // V enters P.V as fp16
                            a0 = f32_to_f16_bits(bf16_bits_to_f32(a0));
                            a1 = f32_to_f16_bits(bf16_bits_to_f32(a1));
                        }
                        const int d = ch * 8 + j;
                        *(uint32_t *) &Vt[buf][d * LSTR + kp] = (uint32_t) a0 | ((uint32_t) a1 << 16);
                    }
                }
            }
        }
    };

    const bool has_mask = p.mask != nullptr, has_rel = p.rel_lut != nullptr;
    const char *mrow[QB];
    const float *rrow[QB];     // relative bias: rrow[qb][key] = lut value of (key - qrow)
    for (int qb = 0; qb < QB; ++qb) {
        const int qrow = qbase + qb * 16 + lr;
        const int qr = qrow < p.Nq ? qrow : 0;
        mrow[qb] = has_mask ? (const char *) p.mask + (int64_t) qr * p.m_nb1 +
                                  (int64_t) (h % p.m_ne2) * p.m_nb2 + (int64_t) (b % p.m_ne3) * p.m_nb3
                            : nullptr;
        rrow[qb] = has_rel ? p.rel_lut + (int64_t) h * p.rel_nh + p.rel_off - qr : nullptr;
    }

    // tiles past the last key load zeros and are masked like keys >= Nkv
    gload(ks);
    lstore(0);
    __syncthreads();

    for (int it = 0; it < niter; ++it) {
        const int buf = it & 1;
        if (it + 1 < niter) gload((it + 1) * KS + ks);
        const int k0 = (it * KS + ks) * KT;

        // ---- S^T = K . Q^T : s[qb][t][r] = S^T[key = k0+16t+4lg+r][q = lr]
        f32x4 s[QB][4];
        for (int qb = 0; qb < QB; ++qb)
            for (int t = 0; t < 4; ++t) s[qb][t] = f32x4{0, 0, 0, 0};
        if constexpr (F32) {
            for (int t = 0; t < 4; ++t)
                for (int kc = 0; kc < 16; ++kc) {
                    const float a = Ks[buf][(16 * t + lr) * LSTR + 4 * kc + lg];
                    for (int qb = 0; qb < QB; ++qb)
                        s[qb][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, qf32[qb][kc], s[qb][t], 0, 0, 0);
                }
        } else {
            for (int t = 0; t < 4; ++t)
                for (int kc = 0; kc < 2; ++kc) {
                    const frag16 a = *(const frag16 *) &Ks[buf][(16 * t + lr) * LSTR + 32 * kc + 8 * lg];
                    for (int qb = 0; qb < QB; ++qb) {
                        if constexpr (KVE == Elt::BF16)
                            s[qb][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf16[qb][kc], s[qb][t], 0, 0, 0);
                        else
                            s[qb][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf16[qb][kc], s[qb][t], 0, 0, 0);
                    }
                }
        }

        // ---- online softmax (base 2): x = s*scale*log2e (+ softcap, mask)
        float pv[QB][4][4];
        for (int qb = 0; qb < QB; ++qb) {
            float mloc = -INFINITY;
            for (int t = 0; t < 4; ++t)
                for (int r = 0; r < 4; ++r) {
                    const int key = k0 + 16 * t + 4 * lg + r;
                    float x = s[qb][t][r];
                    if (p.softcap != 0.0f) x = p.softcap * tanhf(x * p.scale);
                    else x = x * p.scale;
                    if (has_mask && key < p.Nkv) {
                        const float mv = p.mask_f16 ? f16_bits_to_f32(((const uint16_t *) mrow[qb])[key])
                                                    : ((const float *) mrow[qb])[key];
                        x += slope * mv;
                    } else if (has_rel && key < p.Nkv) {
                        const float mv = rrow[qb][key] + (p.key_valid[key] ? 0.0f : -INFINITY);
                        x += slope * mv;
                    }
                    x *= 1.4426950408889634f;             // log2(e)
                    if (key >= p.Nkv) x = -INFINITY;
                    pv[qb][t][r] = x;
                    mloc = fmaxf(mloc, x);
                }
            mloc = half_pair_max(row_pair_max(mloc));       // lanes l ^ 16, l ^ 32 (no LDS)
            const float m_new = fmaxf(m_run[qb], mloc);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_use);
            float lsum = 0.0f;
            for (int t = 0; t < 4; ++t)
                for (int r = 0; r < 4; ++r) {
                    const float e = __builtin_amdgcn_exp2f(pv[qb][t][r] - m_use);
                    pv[qb][t][r] = e;
                    lsum += e;
                }
            l_run[qb] = l_run[qb] * alpha + lsum;
            m_run[qb] = m_new;
            for (int dt = 0; dt < 4; ++dt) oacc[qb][dt] *= alpha;
        }

        // ---- O^T += V^T . P^T
        if constexpr (F32) {
            for (int dt = 0; dt < 4; ++dt)
                for (int t = 0; t < 4; ++t)
                    for (int r = 0; r < 4; ++r) {
                        const float a = Vt[buf][(16 * dt + lr) * LSTR + 16 * t + 4 * lg + r];
                        for (int qb = 0; qb < QB; ++qb)
                            oacc[qb][dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, pv[qb][t][r], oacc[qb][dt], 0, 0, 0);
                    }
        } else {
            f16x8 pb[QB][2];
            for (int qb = 0; qb < QB; ++qb)
                for (int c = 0; c < 2; ++c)
                    for (int j = 0; j < 8; ++j)
                        pb[qb][c][j] = (_Float16) pv[qb][2 * c + (j >> 2)][j & 3];
            for (int dt = 0; dt < 4; ++dt)
                for (int c = 0; c < 2; ++c) {
                    const uint16_t *vr = &Vt[buf][(16 * dt + lr) * LSTR + 32 * c + 4 * lg];
                    const u32x2 lo = *(const u32x2 *) vr;
                    const u32x2 hi = *(const u32x2 *) (vr + 16);
                    u32x4 raw = {lo[0], lo[1], hi[0], hi[1]};
                    f16x8 a;
                    __builtin_memcpy(&a, &raw, 16);
                    for (int qb = 0; qb < QB; ++qb)
                        oacc[qb][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pb[qb][c], oacc[qb][dt], 0, 0, 0);
                }
        }

        if (it + 1 < niter) lstore(buf ^ 1);
        __syncthreads();
    }

    if constexpr (KS > 1) {
        // ranges 1.. leave (m, l, O^T) per lane in their K buffers (every read
        // of them ended at the loop's last barrier); range 0
        // rescales both to the larger max and adds
        constexpr int PER = QB * 18;
        static_assert(NT * PER * sizeof(float) <= sizeof(Ks_all[0]), "merge buffer");
        if (ks > 0) {
            float *st = (float *) Ks_all[ks] + tid;
            for (int qb = 0; qb < QB; ++qb) {
                st[(qb * 18) * NT] = m_run[qb];
                st[(qb * 18 + 1) * NT] = l_run[qb];
                for (int dt = 0; dt < 4; ++dt)
                    for (int r = 0; r < 4; ++r) st[(qb * 18 + 2 + 4 * dt + r) * NT] = oacc[qb][dt][r];
            }
        }
        __syncthreads();
        if (ks > 0) return;
        for (int o = 1; o < KS; ++o) {
            const float *st = (const float *) Ks_all[o] + tid;
            for (int qb = 0; qb < QB; ++qb) {
                const float m1 = st[(qb * 18) * NT], l1 = st[(qb * 18 + 1) * NT];
                const float m = fmaxf(m_run[qb], m1);
                const float mu = m == -INFINITY ? 0.0f : m;
                const float a0 = __builtin_amdgcn_exp2f(m_run[qb] - mu), a1 = __builtin_amdgcn_exp2f(m1 - mu);
                l_run[qb] = l_run[qb] * a0 + l1 * a1;
                m_run[qb] = m;
                for (int dt = 0; dt < 4; ++dt)
                    for (int r = 0; r < 4; ++r)
                        oacc[qb][dt][r] = oacc[qb][dt][r] * a0 + st[(qb * 18 + 2 + 4 * dt + r) * NT] * a1;
            }
        }
    }

    // ---------------- epilogue: O = O^T / l, dst ne = [D, H, Nq, B]
    for (int qb = 0; qb < QB; ++qb) {
        float l = l_run[qb];
        l = half_pair_sum(row_pair_sum(l));
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        const int qrow = qbase + qb * 16 + lr;
        if (qrow >= p.Nq) continue;
        char *orow = (char *) p.o + (int64_t) b * p.o_nb3 + (int64_t) qrow * p.o_nb2 + (int64_t) h * p.o_nb1;
        for (int dt = 0; dt < 4; ++dt) {
            const int d0 = 16 * dt + 4 * lg;
            if constexpr (OE == Elt::F32) {
                f32x4 v = oacc[qb][dt] * inv;
                *(f32x4 *) (orow + d0 * 4) = v;
            } else {
                uint16_t t4[4];
                for (int r = 0; r < 4; ++r) t4[r] = f32_to_bf16_bits(oacc[qb][dt][r] * inv);
                u32x2 w;
                __builtin_memcpy(&w, t4, 8);
                *(u32x2 *) (orow + d0 * 2) = w;
            }
        }
    }
}

template <Elt QE, Elt KVE, Elt OE>
hipError_t launch_attn_t(const AttnParams &p, hipStream_t s) {
    // 4 waves x 1 block of 16 rows when few rows, else 4 waves x 2 blocks
    const int rows_per_wg_big = 4 * 2 * 16;
    const int64_t wgs_big = (int64_t) ((p.Nq + rows_per_wg_big - 1) / rows_per_wg_big) * p.H * p.B;
    const int64_t wgs_small = (int64_t) ((p.Nq + 63) / 64) * p.H * p.B;
    // F32 K/V on at most one workgroup per CU: two key ranges per workgroup
    // (139 KiB of static LDS), so two waves share each SIMD; only where the
    // device gives a workgroup that much LDS
    constexpr size_t ks2_lds = sizeof(float) * 2 * 2 * (KT * LDS32 + D * LDS32);
    const DeviceInfo &dev = device_info();
    if (KVE == Elt::F32 && wgs_small <= dev.cus && dev.lds_per_block >= ks2_lds) {
        dim3 grid((p.Nq + 63) / 64, p.H, p.B);
        launch_kernel((attn_kernel<QE, KVE, OE, 4, 1, 2>), grid, dim3(512), 0, s, p);
    } else if (KVE != Elt::F32 && wgs_big >= 256) {
        dim3 grid((p.Nq + rows_per_wg_big - 1) / rows_per_wg_big, p.H, p.B);
        launch_kernel((attn_kernel<QE, KVE, OE, 4, 2>), grid, dim3(256), 0, s, p);
    } else {
        constexpr int rows = 4 * 1 * 16;
        dim3 grid((p.Nq + rows - 1) / rows, p.H, p.B);
        launch_kernel((attn_kernel<QE, KVE, OE, 4, 1>), grid, dim3(256), 0, s, p);
    }
    return hipGetLastError();
}

template <Elt QE, Elt KVE>
hipError_t launch_attn_o(const AttnParams &p, hipStream_t s) {
    return p.out_bf16 ? launch_attn_t<QE, KVE, Elt::BF16>(p, s) : launch_attn_t<QE, KVE, Elt::F32>(p, s);
}

template <Elt KVE>
hipError_t launch_attn_q(const AttnParams &p, hipStream_t s) {
    switch (p.q_type) {
        case TSK_TYPE_F32:  return launch_attn_o<Elt::F32, KVE>(p, s);
        case TSK_TYPE_F16:  return launch_attn_o<Elt::F16, KVE>(p, s);
        default:            return launch_attn_o<Elt::BF16, KVE>(p, s);
    }
}

}  // namespace

hipError_t launch_attention(const AttnParams &p, hipStream_t s) {
    switch (p.kv_type) {
        case TSK_TYPE_F32: return launch_attn_q<Elt::F32>(p, s);
        case TSK_TYPE_F16: return launch_attn_q<Elt::F16>(p, s);
        default:           return launch_attn_q<Elt::BF16>(p, s);
    }
}

}  // namespace tsk
