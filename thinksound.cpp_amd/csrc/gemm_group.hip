// gemm_group.hip — BF16 weight GEMMs of the MM-DiT block projections on gfx950
// (the ggml_mul_mat nodes of lin(), src/mmdit.cpp:12-25), one launch for up to
// two independent problems (the latent and text streams of a joint block).
//
//   Y[n, m] = epi( sum_k X[n, k] * W[m, k] + bias[m] )
//
// The projections are thin: N = 154..1446 tokens against M x K = 1024..4096
// squared weights, so the chip is filled along the weight rows and every
// weight element is read by only ceil(N / BN) workgroups. A workgroup keeps
// its whole activation tile [BN tokens][K chunk] resident in LDS (loaded once,
// converted to bf16 on the way in), and each of its four waves streams ITS OWN
// weight rows straight from global memory into MFMA A-operand registers,
// PF K-steps ahead. The weight tile needs no LDS staging (no wave shares it)
// and the main loop has no barrier.
//
// bf16 MFMA 16x16x32, fp32 accumulation: A = 16 weight rows, B = 16 tokens, so
// a lane ends with 4 consecutive output features of one token.
//
// Epilogues: f32 / bf16 store (+bias), GELU(tanh) -> bf16, split-K partial
// slices (summed in fixed order by the consumer, so results do not depend on
// the launch shape), the QKV epilogue that applies RMSNorm*w to q and k,
// RoPE on the latent stream and the F16 cast into the attention layout
// [B][n_head][Ntot][64] (mmdit.cpp:80-90), through an LDS transpose, and
// SwiGLU: half of a wave's weight tiles stream W1 rows, the other half the
// same rows of W3, so each lane holds h1 and h3 of the same (feature, token)
// and writes silu(h1) * h3 (convmlp / mlp, mmdit.cpp:39-52).
//
// Convolutions (conv1d_f32 / conv_cl, mmdit.cpp:20-34) run as this GEMM with
// K = KW * IC over an implicit im2col: the activation tile is gathered from
// shifted position rows of the channels-fastest input while it is staged
// into LDS, so no im2col buffer exists. This needs the weight's K in
// kw-major order (k = kw * IC + ic), a load-time permutation of ggml's
// [KW, IC, OC] kernel (k = ic * KW + kw); only the order of the fp32
// accumulation differs from the ggml graph.
#include "tsk_common.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

namespace tsk {

namespace {

constexpr int NT = 256;       // 4 waves
constexpr int KS = 64;        // K per main-loop step: two MFMAs per (A, B) tile pair
constexpr int KCMAX = 1024;   // activation K resident in LDS per chunk (filled in 2 x 512 columns)

template <int TM, int TN>
struct Tile {
    static constexpr int BM = 4 * TM * 16;   // weight rows (output features) per workgroup
    static constexpr int BN = TN * 16;       // tokens per workgroup
};

// Workgroup -> (problem, m tile, n tile, split). Problems start at multiples of
// 8 so that bid % 8 (the XCD the workgroup lands on) is the same in both
// numberings; when the m tiles split evenly over the 8 XCDs, all workgroups
// reading one weight tile go to the same XCD and share its L2.
struct TileCoord {
    int pi, tm, tn, split;
};
__device__ __forceinline__ bool decode(const GemmGroup &g, TileCoord &c) {
    const int bid = blockIdx.x;
    c.pi = (g.nprob > 1 && bid >= g.p[1].block_begin) ? 1 : 0;
    const GemmProblem &p = g.p[c.pi];
    const int li = bid - p.block_begin;
    const int cols = p.tiles_n * p.splits;
    if (li >= p.tiles_m * cols) return false;
    int col;
    if ((p.tiles_m & 7) == 0) {
        const int s = li >> 3;
        c.tm = (li & 7) + 8 * (s / cols);
        col = s % cols;
    } else {
        c.tm = li % p.tiles_m;
        col = li / p.tiles_m;
    }
    c.tn = col % p.tiles_n;
    c.split = col / p.tiles_n;
    return true;
}

__device__ __forceinline__ int64_t x_row_offset(const GemmProblem &p, int n) {
    return p.x_group_rows ? (int64_t) (n / p.x_group_rows) * p.x_group_stride + (int64_t) (n % p.x_group_rows) * p.ld_x
                          : (int64_t) n * p.ld_x;
}

constexpr bool is_swiglu(int epi) { return epi == EPI_SWIGLU_F32 || epi == EPI_SWIGLU_BF16; }

template <int TM, int TN, int PF, bool XF32, int EPI>
__global__ __launch_bounds__(NT) void gemm_group_kernel(const GemmGroup g, int KC) {
    extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
    constexpr int BM = Tile<TM, TN>::BM, BN = Tile<TM, TN>::BN;
    constexpr bool SWIGLU = is_swiglu(EPI);
    constexpr int TMO = SWIGLU ? TM / 2 : TM;     // output row tiles per wave
    constexpr int BMO = 4 * TMO * 16;             // output features per workgroup
    static_assert(PF * TM * 2 <= 48, "vmcnt range");
    static_assert(!SWIGLU || TM % 2 == 0, "SwiGLU pairs weight tiles");

    TileCoord tc;
    if (!decode(g, tc)) return;
    const GemmProblem &p = g.p[tc.pi];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int bm0 = tc.tm * BMO, bn0 = tc.tn * BN;
    const int LDX = KC + 8;                       // bf16 per LDS row: 16-B pad against bank conflicts
    const int kspl = ((p.K + p.splits - 1) / p.splits + KS - 1) / KS * KS;
    const int kbeg = tc.split * kspl, kend = min(p.K, kbeg + kspl);

    // this lane's weight rows (A operand: row lr of each 16-row tile). Rows past
    // M read row 0: their outputs are never stored, so no select is needed and
    // every load in the main loop is unconditional (static vmcnt bookkeeping
    // keeps PF steps in flight).
    // Row-major weights: piece 0 of K-step s sits at wrow + c0 + 8 lg + 64 s,
    // piece 1 at +32; tiled weights: the lane's 16 B of tile (rb, k / 32) at
    // wrow + (k / 32) * 512 (lane offset folded into wrow), piece 1 at +512.
    // Pieces outside [c0, c1) load offset 0 instead (a valid address).
    // SwiGLU: tiles [0, TMO) are W1's row blocks, [TMO, TM) the same of W3.
    const uint16_t *wrow[TM];
    for (int i = 0; i < TM; ++i) {
        const int rb = (bm0 >> 4) + wave * TMO + i % TMO;
        const uint16_t *wb = SWIGLU && i >= TMO ? p.w3 : p.w;
        if (p.w_tiled) {
            wrow[i] = wb + (int64_t) min(rb, p.M / 16 - 1) * (p.K / 32) * 512 + lane * 8;
        } else {
            const int row = rb * 16 + lr;
            wrow[i] = wb + (int64_t) (row < p.M ? row : 0) * p.ld_w;
        }
    }
    const int wstep = p.w_tiled ? 1024 : 64, wpiece = p.w_tiled ? 512 : 32;

    f32x4 acc[TM][TN];
    for (int i = 0; i < TM; ++i)
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    u32x4 wr[PF][TM][2];

    for (int c0 = kbeg; c0 < kend; c0 += KC) {
        const int c1 = min(kend, c0 + KC);
        const int nst = (c1 - c0 + KS - 1) / KS;
        const bool ragged = (c1 - c0) % KS != 0;     // last step ends inside a 64-wide step
        // K-step `step` of this chunk: lane group lg holds k = 8 lg + [0, 8) of
        // each 32-wide half (the MFMA's own operand layout). K % 8 == 0, so a
        // 16-B piece is wholly inside or wholly outside [c0, c1); outside
        // pieces load row start instead and are zeroed when used.
        const int64_t wc0 = p.w_tiled ? (int64_t) (c0 / 32) * 512 : c0 + 8 * lg;
        auto wload = [&](int st, int step) {
            const int k = c0 + step * KS + 8 * lg;
            const int64_t o0 = wc0 + (int64_t) step * wstep;
            const int64_t k0 = k < c1 ? o0 : 0, k1 = k + 32 < c1 ? o0 + wpiece : 0;
            for (int i = 0; i < TM; ++i) {
                wr[st][i][0] = *(const u32x4 *) (wrow[i] + k0);
                wr[st][i][1] = *(const u32x4 *) (wrow[i] + k1);
            }
        };
        auto compute = [&](int st, int step) {
            const int kx = step * KS + 8 * lg;
            bf16x8 b0[TN], b1[TN];
            for (int j = 0; j < TN; ++j) {
                const uint16_t *xr = xs + (j * 16 + lr) * LDX + kx;
                b0[j] = *(const bf16x8 *) xr;
                b1[j] = *(const bf16x8 *) (xr + 32);
            }
            const bool mask = ragged && step == nst - 1;   // wave-uniform
            const bool ok0 = c0 + kx < c1, ok1 = c0 + kx + 32 < c1;
            for (int i = 0; i < TM; ++i) {
                u32x4 w0 = wr[st][i][0], w1 = wr[st][i][1];
                if (mask) {
                    w0 = ok0 ? w0 : u32x4{0, 0, 0, 0};
                    w1 = ok1 ? w1 : u32x4{0, 0, 0, 0};
                }
                const bf16x8 a0 = __builtin_bit_cast(bf16x8, w0);
                const bf16x8 a1 = __builtin_bit_cast(bf16x8, w1);
                for (int j = 0; j < TN; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[j], acc[i][j], 0, 0, 0);
                }
            }
        };

        // activation tile [BN][nst * KS] -> LDS as bf16, zero past N and c1.
        // Wave w fills rows w, w + 4, ... (wave-uniform row offsets); lanes
        // cover 8 columns each, KCMAX = 1024 columns in 2 passes. The tile's
        // loads are issued before the first PF weight steps (bf16 activations),
        // so the stores wait only for them (vmcnt retires in order).
        constexpr int RPW = BN / 4;                   // rows per wave
        static_assert(2 * RPW <= 32, "piece mask");
        const int kcr = nst * KS;
        const int wv = __builtin_amdgcn_readfirstlane(wave);
        u32x4 xv[RPW][2][XF32 ? 2 : 1];
        uint32_t xok = 0;                             // bit 2 g2 + h: the piece holds data
        auto xload = [&]() {
#pragma unroll
            for (int g2 = 0; g2 < RPW; ++g2) {
                const int r = wv + 4 * g2;
                const bool rok = bn0 + r < p.N;
                const int n = rok ? bn0 + r : 0;
                int64_t roff;
                int iw0 = 0;
                if (p.conv_ic) {
                    // output position ow of batch item b reads input positions
                    // ow * s + kw * d - p
                    const int b = n / p.conv_ow, ow = n - b * p.conv_ow;
                    roff = (int64_t) b * p.x_group_stride;
                    iw0 = ow * p.conv_s - p.conv_p;
                } else {
                    roff = x_row_offset(p, n);
                }
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int col = lane * 8 + 512 * h;
                    const int k = c0 + col;
                    bool ok = rok && k < c1;
                    int64_t off;
                    if (p.conv_ic) {
                        const int kw = k / p.conv_ic, ic = k - kw * p.conv_ic;
                        const int iw = iw0 + kw * p.conv_d;
                        ok = ok && iw >= 0 && iw < p.conv_iw;
                        off = ok ? roff + (int64_t) iw * p.ld_x + ic : 0;
                    } else {
                        off = roff + (ok ? k : 0);
                    }
                    xok |= (uint32_t) ok << (2 * g2 + h);
                    if constexpr (XF32) {
                        const float *xf = (const float *) p.x + off;
                        xv[g2][h][0] = *(const u32x4 *) xf;
                        xv[g2][h][1] = *(const u32x4 *) (xf + 4);
                    } else {
                        xv[g2][h][0] = *(const u32x4 *) ((const uint16_t *) p.x + off);
                    }
                }
            }
        };
        auto xstore = [&]() {
#pragma unroll
            for (int g2 = 0; g2 < RPW; ++g2) {
                const int r = wv + 4 * g2;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int col = lane * 8 + 512 * h;
                    const bool ok = (xok >> (2 * g2 + h)) & 1;
                    u32x4 t;
                    if constexpr (XF32) {
                        const float *f0 = (const float *) &xv[g2][h][0], *f1 = (const float *) &xv[g2][h][1];
                        uint16_t t8[8];
                        for (int e = 0; e < 4; ++e) { t8[e] = f32_to_bf16_bits(f0[e]); t8[4 + e] = f32_to_bf16_bits(f1[e]); }
                        __builtin_memcpy(&t, t8, 16);
                    } else {
                        t = xv[g2][h][0];
                    }
                    if (col < kcr) *(u32x4 *) &xs[r * LDX + col] = ok ? t : u32x4{0, 0, 0, 0};
                }
            }
        };
        xok = 0;
        xload();
        if constexpr (XF32) {
            xstore();     // f32 tiles hold twice the registers: store before the weights go out
            for (int st = 0; st < PF; ++st) wload(st, min(st, nst - 1));
        } else {
            for (int st = 0; st < PF; ++st) wload(st, min(st, nst - 1));
            xstore();
        }
        __syncthreads();

        int s = 0;
        for (; s + PF <= nst; s += PF) {
#pragma unroll
            for (int st = 0; st < PF; ++st) {
                compute(st, s + st);
                wload(st, min(s + st + PF, nst - 1));
            }
        }
#pragma unroll
        for (int st = 0; st < PF; ++st)
            if (s + st < nst) compute(st, s + st);
        if (c1 < kend) __syncthreads();              // the next chunk overwrites the tile
    }

    // ------------------------------------------------------------ epilogues
    if constexpr (EPI == EPI_QKV) {
        // acc + bias -> LDS [BN][BM] f32, then one 16-lane group per (token, head)
        constexpr int LDY = BM + 4;
        float *ys = (float *) xs;
        __syncthreads();
        for (int i = 0; i < TM; ++i) {
            const int ml = (wave * TM + i) * 16 + 4 * lg;
            const int m0 = bm0 + ml;
            f32x4 bv = f32x4{0, 0, 0, 0};
            if (p.bias && m0 < p.M) bv = *(const f32x4 *) (p.bias + m0);
            for (int j = 0; j < TN; ++j) {
                const f32x4 v = acc[i][j];
                *(f32x4 *) &ys[(j * 16 + lr) * LDY + ml] = f32x4{v[0] + bv[0], v[1] + bv[1], v[2] + bv[2], v[3] + bv[3]};
            }
        }
        __syncthreads();
        const int H = p.M / 3, nh = H / 64;
        const int grp = tid >> 4, sl = tid & 15;
        constexpr int HPT = BM / 64;                 // heads per tile
        for (int pp = grp; pp < BN * HPT; pp += NT / 16) {
            const int nl = pp / HPT, hl = pp % HPT;
            const int n = bn0 + nl, f0 = bm0 + hl * 64;
            const bool live = n < p.N && f0 < p.M;
            f32x4 x = *(const f32x4 *) &ys[nl * LDY + hl * 64 + 4 * sl];
            const int sec = f0 / H, head = (f0 % H) / 64;
            const int b = (live ? n : 0) / p.seq, spos = (live ? n : 0) % p.seq;
            if (sec < 2) {
                const float ss = row16_sum(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);   // one DPP row
                const float sc = 1.0f / sqrtf(ss / 64.0f + p.eps);
                const float *w = sec ? p.kn_w : p.qn_w;
                const f32x4 wv = *(const f32x4 *) (w + 4 * sl);
                for (int e = 0; e < 4; ++e) x[e] = x[e] * sc * wv[e];
                if (p.rope) {
                    for (int q2 = 0; q2 < 2; ++q2) {
                        const float th = p.freq_scale * rope_theta((float) spos, p.theta_scale, 2 * sl + q2);
                        const float cs = cosf(th), sn = sinf(th);
                        const float x0 = x[2 * q2], x1 = x[2 * q2 + 1];
                        x[2 * q2] = x0 * cs - x1 * sn;
                        x[2 * q2 + 1] = x0 * sn + x1 * cs;
                    }
                }
            }
            if (live) {
                if (sec == 0)
                    for (int e = 0; e < 4; ++e) x[e] *= p.q_scale;     // the attention's softmax scale
                uint16_t o4[4] = {f32_to_f16_bits(x[0]), f32_to_f16_bits(x[1]), f32_to_f16_bits(x[2]), f32_to_f16_bits(x[3])};
                if (sec < 2) {
                    u32x2 w2;
                    __builtin_memcpy(&w2, o4, 8);
                    *(u32x2 *) ((sec ? p.k : p.q) + (((int64_t) b * nh + head) * p.Ntot + p.tok_off + spos) * 64 + 4 * sl) = w2;
                } else {
                    uint16_t *vcol = p.vt + (((int64_t) b * nh + head) * 64 + 4 * sl) * p.ldv + vt_pos(p.tok_off + spos);
                    for (int e = 0; e < 4; ++e) vcol[(int64_t) e * p.ldv] = o4[e];
                }
            }
        }
        return;
    } else if constexpr (SWIGLU) {
        for (int i = 0; i < TMO; ++i) {
            const int m0 = bm0 + (wave * TMO + i) * 16 + 4 * lg;
            if (m0 >= p.M) continue;
            const bool full = m0 + 3 < p.M;
            for (int j = 0; j < TN; ++j) {
                const int n = bn0 + j * 16 + lr;
                if (n >= p.N) continue;
                float o[4];
                for (int r = 0; r < 4; ++r) {
                    const float h1 = acc[i][j][r], h3 = acc[i + TMO][j][r];
                    o[r] = h1 * __builtin_amdgcn_rcpf(1.0f + __expf(-h1)) * h3;   // silu: the cooperative tiles' form
                }
                if constexpr (EPI == EPI_SWIGLU_BF16) {
                    uint16_t *yr = (uint16_t *) p.y + (int64_t) n * p.ld_y + m0;
                    if (full) {
                        uint16_t t4[4];
                        for (int r = 0; r < 4; ++r) t4[r] = f32_to_bf16_bits(o[r]);
                        u32x2 w;
                        __builtin_memcpy(&w, t4, 8);
                        *(u32x2 *) yr = w;
                    } else {
                        for (int r = 0; r < 4 && m0 + r < p.M; ++r) yr[r] = f32_to_bf16_bits(o[r]);
                    }
                } else {
                    float *yr = (float *) p.y + (int64_t) n * p.ld_y + m0;
                    if (full) *(f32x4 *) yr = f32x4{o[0], o[1], o[2], o[3]};
                    else for (int r = 0; r < 4 && m0 + r < p.M; ++r) yr[r] = o[r];
                }
            }
        }
    } else {
        for (int i = 0; i < TM; ++i) {
            const int m0 = bm0 + (wave * TM + i) * 16 + 4 * lg;
            if (m0 >= p.M) continue;
            const bool full = m0 + 3 < p.M;
            float bv[4] = {0.f, 0.f, 0.f, 0.f};
            if (EPI != EPI_PARTIAL && p.bias) {
                if (full) { const f32x4 t = *(const f32x4 *) (p.bias + m0); bv[0] = t[0]; bv[1] = t[1]; bv[2] = t[2]; bv[3] = t[3]; }
                else for (int r = 0; r < 4 && m0 + r < p.M; ++r) bv[r] = p.bias[m0 + r];
            }
            for (int j = 0; j < TN; ++j) {
                const int n = bn0 + j * 16 + lr;
                if (n >= p.N) continue;
                float o[4];
                for (int r = 0; r < 4; ++r) o[r] = acc[i][j][r] + bv[r];
                if constexpr (EPI == EPI_GELU_BF16)
                    for (int r = 0; r < 4; ++r) o[r] = gelu_tanh_f(o[r]);
                if constexpr (EPI == EPI_STORE_BF16 || EPI == EPI_GELU_BF16) {
                    uint16_t *yr = (uint16_t *) p.y + (int64_t) n * p.ld_y + m0;
                    if (full) {
                        uint16_t t4[4];
                        for (int r = 0; r < 4; ++r) t4[r] = f32_to_bf16_bits(o[r]);
                        u32x2 w;
                        __builtin_memcpy(&w, t4, 8);
                        *(u32x2 *) yr = w;
                    } else {
                        for (int r = 0; r < 4 && m0 + r < p.M; ++r) yr[r] = f32_to_bf16_bits(o[r]);
                    }
                } else {
                    float *yr = (float *) p.y + (EPI == EPI_PARTIAL ? (int64_t) tc.split * p.N * p.ld_y : 0) +
                                (int64_t) n * p.ld_y + m0;
                    if (full) *(f32x4 *) yr = f32x4{o[0], o[1], o[2], o[3]};
                    else for (int r = 0; r < 4 && m0 + r < p.M; ++r) yr[r] = o[r];
                }
            }
        }
    }
}

template <int TM, int TN, int PF, bool XF32, int EPI>
hipError_t launch_cfg(const GemmGroup &g, int KC, int nblocks, size_t lds, hipStream_t s) {
    auto kern = gemm_group_kernel<TM, TN, PF, XF32, EPI>;
    lds_opt_in((const void *) kern, lds);
    launch_kernel(kern, dim3(nblocks), dim3(NT), lds, s, g, KC);
    return hipGetLastError();
}

template <int TM, int TN, int PF>
hipError_t group_launch(GemmGroup &g, int flags, int epi, hipStream_t s) {
    constexpr int BM = Tile<TM, TN>::BM, BN = Tile<TM, TN>::BN;
    if (g.nprob < 1 || g.nprob > 2) return hipErrorInvalidValue;
    const bool xf32 = (flags & GEMM_X_F32) != 0;
    const bool swiglu = is_swiglu(epi);
    if (xf32 && epi != EPI_STORE_F32 && epi != EPI_STORE_BF16 && !swiglu) return hipErrorInvalidValue;
    const int bmo = swiglu ? BM / 2 : BM;
    // K held in LDS per chunk: up to KCMAX, within the device's LDS per workgroup
    const int kc_dev = min(KCMAX, ((int) device_lds_per_block() / (2 * BN) - 8) / KS * KS);
    if (kc_dev < KS) return hipErrorInvalidConfiguration;
    int nblocks = 0, kc = KS;
    for (int i = 0; i < g.nprob; ++i) {
        GemmProblem &p = g.p[i];
        if (p.M < 1 || p.N < 1 || p.K < 8 || (p.K & 7) || p.splits < 1) return hipErrorInvalidValue;
        if (epi != EPI_PARTIAL && p.splits != 1) return hipErrorInvalidValue;
        if (epi == EPI_QKV && (p.M % 192 || p.seq < 1)) return hipErrorInvalidValue;
        if (p.w_tiled && (p.M % 16 || p.K % 32)) return hipErrorInvalidValue;
        if (swiglu && (!p.w3 || p.bias)) return hipErrorInvalidValue;
        if (p.conv_ic) {
            // every 16-B piece of a K step lies inside one kw slice
            if (p.conv_ic % 8 || p.K % p.conv_ic || p.x_group_rows || p.conv_ow < 1 || p.conv_iw < 1 ||
                p.conv_s < 1 || p.conv_d < 1 || p.conv_p < 0 || p.N % p.conv_ow)
                return hipErrorInvalidValue;
        }
        p.tiles_m = (p.M + bmo - 1) / bmo;
        p.tiles_n = (p.N + BN - 1) / BN;
        p.block_begin = (nblocks + 7) & ~7;
        nblocks = p.block_begin + p.tiles_m * p.tiles_n * p.splits;
        const int kspl = ((p.K + p.splits - 1) / p.splits + KS - 1) / KS * KS;
        kc = max(kc, min(kc_dev, kspl));
    }
    size_t lds = (size_t) BN * (kc + 8) * 2;
    if (epi == EPI_QKV) lds = max(lds, (size_t) BN * (BM + 4) * 4);
    switch (epi) {
        case EPI_STORE_F32:
            return xf32 ? launch_cfg<TM, TN, PF, true, EPI_STORE_F32>(g, kc, nblocks, lds, s)
                        : launch_cfg<TM, TN, PF, false, EPI_STORE_F32>(g, kc, nblocks, lds, s);
        case EPI_STORE_BF16:
            return xf32 ? launch_cfg<TM, TN, PF, true, EPI_STORE_BF16>(g, kc, nblocks, lds, s)
                        : launch_cfg<TM, TN, PF, false, EPI_STORE_BF16>(g, kc, nblocks, lds, s);
        case EPI_GELU_BF16: return launch_cfg<TM, TN, PF, false, EPI_GELU_BF16>(g, kc, nblocks, lds, s);
        case EPI_QKV: return launch_cfg<TM, TN, PF, false, EPI_QKV>(g, kc, nblocks, lds, s);
        case EPI_PARTIAL: return launch_cfg<TM, TN, PF, false, EPI_PARTIAL>(g, kc, nblocks, lds, s);
        case EPI_SWIGLU_F32:
            return xf32 ? launch_cfg<TM, TN, PF, true, EPI_SWIGLU_F32>(g, kc, nblocks, lds, s)
                        : launch_cfg<TM, TN, PF, false, EPI_SWIGLU_F32>(g, kc, nblocks, lds, s);
        case EPI_SWIGLU_BF16:
            return xf32 ? launch_cfg<TM, TN, PF, true, EPI_SWIGLU_BF16>(g, kc, nblocks, lds, s)
                        : launch_cfg<TM, TN, PF, false, EPI_SWIGLU_BF16>(g, kc, nblocks, lds, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_gemm_group(GemmGroup &g, int flags, int epi, hipStream_t s) {
    // 128 x 32 tiles, 4 K-steps in flight; grids of more than ~2.5 tiles per CU
    // (N >= ~1000 tokens) run 256 x 32 tiles. Measured on MI355X over the DiT
    // projection shapes; the tile shape does not change any summation order.
    int64_t tiles = 0;
    for (int i = 0; i < g.nprob; ++i)
        tiles += (int64_t) ((g.p[i].M + 127) / 128) * ((g.p[i].N + 31) / 32) * max(g.p[i].splits, 1);
    if (tiles > 640) return group_launch<4, 2, 3>(g, flags, epi, s);
    return group_launch<2, 2, 4>(g, flags, epi, s);
}

}  // namespace tsk
