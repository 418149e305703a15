// gemm.hip — weight GEMMs of the MM-DiT projections for gfx950
// (ggml_mul_mat nodes of lin() / conv1d_f32(), src/mmdit.cpp:12-25).
//
//   Y[n, m] = epi( sum_k X[n, k] * W[m, k] + bias[m] )
//
// BF16 weights: bf16 MFMA 16x16x32, fp32 accumulation; f32 activations are
// rounded to bf16 (RNE) while staged, which is ggml's conversion of src1 to
// the weight's vec_dot type.
// Q8_0 weights: int8 MFMA 16x16x32 = exactly one 32-element Q8_0 block per
// instruction, so each MFMA yields the exact integer block sum of ggml's
// vec_dot_q8_0_q8_0; it is scaled by fp32(d_w) * fp32(d_x) into fp32
// accumulators. Activations were quantized per 32-block beforehand.
//
// Tiling: workgroup = WM x WN waves; a wave owns TM x TN 16x16 tiles with
// A = W rows (output features) and B = X rows (tokens), so each lane ends up
// with 4 consecutive output features of one token (16-B stores). Operand
// tiles are double buffered through LDS with one barrier per K step.
#include "qkv_row.h"
#include "tsk_common.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

#include <cstdlib>
#include <cstring>

namespace tsk {

namespace {


// 4 floats of row `row` at columns m0 .. m0 + 3 (zeros past M)
__device__ __forceinline__ f32x4 load4_guard(const float *row, int m0, int M) {
    if (m0 + 3 < M) return *(const f32x4 *) (row + m0);
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int r = 0; r < 4 && m0 + r < M; ++r) v[r] = row[m0 + r];
    return v;
}

// Epilogue of a wave's TI x TJ output fragments (lane: features m0[i] .. + 3
// of token n[j]): every load (bias, gate, residual) of all fragments first,
// then one wait the compiler sees, then the stores -- loads and stores share
// one counter, so a load issued behind a store would also wait for it.
template <int EPI, bool YBF16, int TI, int TJ>
__device__ __forceinline__ void epilogue_frags(const GemmParams &p, const int (&m0)[TI], const int (&n)[TJ],
                                               const f32x4 (&acc)[TI][TJ]) {
    f32x4 bv[TI], gv[TI][TJ], rv[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i) bv[i] = p.bias && m0[i] < p.M ? load4_guard(p.bias, m0[i], p.M) : f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (EPI == EPI_GATE_RES) {
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const bool ok = n[j] < p.N && m0[i] < p.M;
                gv[i][j] = ok ? load4_guard(p.gate + (int64_t) (n[j] / p.rows_per_gate) * p.ld_gate, m0[i], p.M)
                              : f32x4{0.f, 0.f, 0.f, 0.f};
                rv[i][j] = ok ? load4_guard(p.res + (int64_t) n[j] * p.ld_res, m0[i], p.M) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
    }
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int mm = m0[i], nn = n[j];
            if (nn >= p.N || mm >= p.M) continue;
            const bool full = mm + 3 < p.M;
            float o[4];
            for (int r = 0; r < 4; ++r) o[r] = acc[i][j][r] + bv[i][r];
            if constexpr (EPI == EPI_GEGLU) {
                // features mm .. mm + 3 are (a_j, b_j, a_j+1, b_j+1), j = mm / 2 (M % 4 == 0)
                float *yr = (float *) p.y + (int64_t) nn * p.ld_y + mm / 2;
                *(f32x2 *) yr = f32x2{gelu_tanh_f(o[0]) * o[1], gelu_tanh_f(o[2]) * o[3]};
                continue;
            }
            if constexpr (EPI == EPI_GELU)
                for (int r = 0; r < 4; ++r) o[r] = gelu_tanh_f(o[r]);
            if constexpr (EPI == EPI_GATE_RES) {
                float *rr = p.res + (int64_t) nn * p.ld_res + mm;
                f32x4 cur = rv[i][j];
                for (int r = 0; r < 4; ++r) cur[r] += gv[i][j][r] * o[r];
                if (full) *(f32x4 *) rr = cur;
                else for (int r = 0; r < 4 && mm + r < p.M; ++r) rr[r] = cur[r];
                continue;
            }
            if constexpr (YBF16) {
                uint16_t *yr = (uint16_t *) p.y + (int64_t) nn * p.ld_y + mm;
                if (full) {
                    uint16_t t4[4];
                    for (int r = 0; r < 4; ++r) t4[r] = f32_to_bf16_bits(o[r]);
                    u32x2 w;
                    __builtin_memcpy(&w, t4, 8);
                    *(u32x2 *) yr = w;
                } else {
                    for (int r = 0; r < 4 && mm + r < p.M; ++r) yr[r] = f32_to_bf16_bits(o[r]);
                }
            } else {
                float *yr = (float *) p.y + (int64_t) nn * p.ld_y + mm;
                if (full) *(f32x4 *) yr = f32x4{o[0], o[1], o[2], o[3]};
                else for (int r = 0; r < 4 && mm + r < p.M; ++r) yr[r] = o[r];
            }
        }
}

// ------------------------------------------------------------------ BF16
constexpr int BK = 64;
constexpr int LDSB = BK + 8;   // bf16 elements per LDS row (144 B)

template <int WM, int WN, int TM, int TN, bool XF32, int EPI, bool YBF16>
__global__ __launch_bounds__(WM * WN * 64)
void gemm_bf16_kernel(const GemmParams p) {
    constexpr int NT = WM * WN * 64;
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    constexpr int WCH = BM * (BK / 8), XCH = BN * (BK / 8);   // 16-B chunks (8 bf16)
    constexpr int WPER = (WCH + NT - 1) / NT, XPER = (XCH + NT - 1) / NT;
    __shared__ __attribute__((aligned(16))) uint16_t Ws[2][BM * LDSB];
    __shared__ __attribute__((aligned(16))) uint16_t Xs[2][BN * LDSB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int wm = wave % WM, wn = wave / WM;
    const int bm0 = blockIdx.x * BM, bn0 = blockIdx.y * BN;
    const uint16_t *W = (const uint16_t *) p.w;

    u32x4 wreg[WPER];
    u32x4 xreg[XPER][XF32 ? 2 : 1];
    const int nk = (p.K + BK - 1) / BK;

    auto gload = [&](int kt) {
        const int k0 = kt * BK;
        for (int i = 0; i < WPER; ++i) {
            const int c = tid + i * NT;
            wreg[i] = u32x4{0, 0, 0, 0};
            if (c < WCH) {
                const int row = bm0 + c / (BK / 8), kk = k0 + (c % (BK / 8)) * 8;
                if (row < p.M && kk < p.K) wreg[i] = *(const u32x4 *) (W + (int64_t) row * p.ld_w + kk);
            }
        }
        for (int i = 0; i < XPER; ++i) {
            const int c = tid + i * NT;
            xreg[i][0] = u32x4{0, 0, 0, 0};
            if constexpr (XF32) xreg[i][1] = u32x4{0, 0, 0, 0};
            if (c < XCH) {
                const int row = bn0 + c / (BK / 8), kk = k0 + (c % (BK / 8)) * 8;
                if (row < p.N && kk < p.K) {
                    const int64_t xoff = p.x_group_rows
                        ? (int64_t) (row / p.x_group_rows) * p.x_group_stride + (int64_t) (row % p.x_group_rows) * p.ld_x
                        : (int64_t) row * p.ld_x;
                    if constexpr (XF32) {
                        const float *xr = (const float *) p.x + xoff + kk;
                        xreg[i][0] = *(const u32x4 *) xr;
                        xreg[i][1] = *(const u32x4 *) (xr + 4);
                    } else {
                        xreg[i][0] = *(const u32x4 *) ((const uint16_t *) p.x + xoff + kk);
                    }
                }
            }
        }
    };
    auto lstore = [&](int buf) {
        for (int i = 0; i < WPER; ++i) {
            const int c = tid + i * NT;
            if (c < WCH) *(u32x4 *) &Ws[buf][(c / (BK / 8)) * LDSB + (c % (BK / 8)) * 8] = wreg[i];
        }
        for (int i = 0; i < XPER; ++i) {
            const int c = tid + i * NT;
            if (c < XCH) {
                u32x4 v;
                if constexpr (XF32) {
                    const float *f0 = (const float *) &xreg[i][0];
                    const float *f1 = (const float *) &xreg[i][1];
                    uint16_t t8[8];
                    for (int j = 0; j < 4; ++j) { t8[j] = f32_to_bf16_bits(f0[j]); t8[4 + j] = f32_to_bf16_bits(f1[j]); }
                    __builtin_memcpy(&v, t8, 16);
                } else {
                    v = xreg[i][0];
                }
                *(u32x4 *) &Xs[buf][(c / (BK / 8)) * LDSB + (c % (BK / 8)) * 8] = v;
            }
        }
    };

    f32x4 acc[TM][TN];
    for (int i = 0; i < TM; ++i)
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
        for (int kk = 0; kk < BK / 32; ++kk) {
            bf16x8 a[TM], b[TN];
            for (int i = 0; i < TM; ++i)
                a[i] = *(const bf16x8 *) &Ws[buf][((wm * TM + i) * 16 + lr) * LDSB + 32 * kk + 8 * lg];
            for (int j = 0; j < TN; ++j)
                b[j] = *(const bf16x8 *) &Xs[buf][((wn * TN + j) * 16 + lr) * LDSB + 32 * kk + 8 * lg];
            for (int i = 0; i < TM; ++i)
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    int m0[TM], nn[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) m0[i] = bm0 + (wm * TM + i) * 16 + 4 * lg;
#pragma unroll
    for (int j = 0; j < TN; ++j) nn[j] = bn0 + (wn * TN + j) * 16 + lr;
    epilogue_frags<EPI, YBF16, TM, TN>(p, m0, nn, acc);
}

// ------------------------------------------------------------------ Q8_0
constexpr int QBK = 128;            // 4 Q8_0 blocks per K step
// block scales of the cooperative Q8_0 tiles are staged in segments of this
// many 32-element blocks (1024 k): 16 KiB of LDS at 64 x 64 tiles, so three
// workgroups fit a CU next to their 2-stage ring
constexpr int Q8_SEG = 32;
constexpr int LDSQ = QBK + 16;      // bytes per LDS row

template <int WM, int WN, int TM, int TN, int EPI, bool YBF16>
__global__ __launch_bounds__(WM * WN * 64)
void gemm_q8_kernel(const GemmParams p) {
    constexpr int NT = WM * WN * 64;
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    constexpr int NBK = QBK / 32;
    constexpr int WCH = BM * (QBK / 16), XCH = BN * (QBK / 16);   // 16-B chunks
    constexpr int WPER = (WCH + NT - 1) / NT, XPER = (XCH + NT - 1) / NT;
    __shared__ __attribute__((aligned(16))) int8_t Wq[2][BM * LDSQ];
    __shared__ __attribute__((aligned(16))) int8_t Xq[2][BN * LDSQ];
    __shared__ float Wd[2][BM * NBK];
    __shared__ float Xd[2][BN * NBK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int wm = wave % WM, wn = wave / WM;
    const int bm0 = blockIdx.x * BM, bn0 = blockIdx.y * BN;
    const int KB = p.K / 32;

    u32x4 wreg[WPER], xreg[XPER];
    float wdreg[(BM * NBK + NT - 1) / NT], xdreg[(BN * NBK + NT - 1) / NT];
    const int nk = (p.K + QBK - 1) / QBK;

    auto gload = [&](int kt) {
        const int k0 = kt * QBK;
        for (int i = 0; i < WPER; ++i) {
            const int c = tid + i * NT;
            wreg[i] = u32x4{0, 0, 0, 0};
            if (c < WCH) {
                const int row = bm0 + c / (QBK / 16), kk = k0 + (c % (QBK / 16)) * 16;
                if (row < p.M && kk < p.K) wreg[i] = *(const u32x4 *) (p.qw + (int64_t) row * p.K + kk);
            }
        }
        for (int i = 0; i < XPER; ++i) {
            const int c = tid + i * NT;
            xreg[i] = u32x4{0, 0, 0, 0};
            if (c < XCH) {
                const int row = bn0 + c / (QBK / 16), kk = k0 + (c % (QBK / 16)) * 16;
                if (row < p.N && kk < p.K) xreg[i] = *(const u32x4 *) (p.qx + (int64_t) row * p.K + kk);
            }
        }
        for (int i = 0; i * NT < BM * NBK; ++i) {
            const int c = tid + i * NT;
            wdreg[i] = 0.0f;
            if (c < BM * NBK) {
                const int row = bm0 + c / NBK, kb = kt * NBK + c % NBK;
                if (row < p.M && kb < KB) wdreg[i] = f16_bits_to_f32(p.dw[(int64_t) row * KB + kb]);
            }
        }
        for (int i = 0; i * NT < BN * NBK; ++i) {
            const int c = tid + i * NT;
            xdreg[i] = 0.0f;
            if (c < BN * NBK) {
                const int row = bn0 + c / NBK, kb = kt * NBK + c % NBK;
                if (row < p.N && kb < KB) xdreg[i] = p.dx[(int64_t) row * KB + kb];
            }
        }
    };
    auto lstore = [&](int buf) {
        for (int i = 0; i < WPER; ++i) {
            const int c = tid + i * NT;
            if (c < WCH) *(u32x4 *) &Wq[buf][(c / (QBK / 16)) * LDSQ + (c % (QBK / 16)) * 16] = wreg[i];
        }
        for (int i = 0; i < XPER; ++i) {
            const int c = tid + i * NT;
            if (c < XCH) *(u32x4 *) &Xq[buf][(c / (QBK / 16)) * LDSQ + (c % (QBK / 16)) * 16] = xreg[i];
        }
        for (int i = 0; i * NT < BM * NBK; ++i) {
            const int c = tid + i * NT;
            if (c < BM * NBK) Wd[buf][c] = wdreg[i];
        }
        for (int i = 0; i * NT < BN * NBK; ++i) {
            const int c = tid + i * NT;
            if (c < BN * NBK) Xd[buf][c] = xdreg[i];
        }
    };

    f32x4 acc[TM][TN];
    for (int i = 0; i < TM; ++i)
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
        for (int kb = 0; kb < NBK; ++kb) {
            long a[TM], b[TN];
            f32x4 dwv[TM];
            float dxv[TN];
            for (int i = 0; i < TM; ++i) {
                const int mr = (wm * TM + i) * 16;
                a[i] = *(const long *) &Wq[buf][(mr + lr) * LDSQ + 32 * kb + 8 * lg];
                for (int r = 0; r < 4; ++r) dwv[i][r] = Wd[buf][(mr + 4 * lg + r) * NBK + kb];
            }
            for (int j = 0; j < TN; ++j) {
                const int nr = (wn * TN + j) * 16;
                b[j] = *(const long *) &Xq[buf][(nr + lr) * LDSQ + 32 * kb + 8 * lg];
                dxv[j] = Xd[buf][(nr + lr) * NBK + kb];
            }
            for (int i = 0; i < TM; ++i)
                for (int j = 0; j < TN; ++j) {
                    const i32x4 isum = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], b[j], i32x4{0, 0, 0, 0}, 0, 0, 0);
                    for (int r = 0; r < 4; ++r)
                        acc[i][j][r] += (float) isum[r] * (dwv[i][r] * dxv[j]);
                }
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    int m0[TM], nn[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) m0[i] = bm0 + (wm * TM + i) * 16 + 4 * lg;
#pragma unroll
    for (int j = 0; j < TN; ++j) nn[j] = bn0 + (wn * TN + j) * 16 + lr;
    epilogue_frags<EPI, YBF16, TM, TN>(p, m0, nn, acc);
}

// ------------------------------------------------------------------ Q8_0, cooperative tiles
// Four waves split a BM x BN tile 2 x 2 and share an LDS ring of 128-k stages
// (four Q8_0 blocks): each 16-row operand unit is 16 rows x 128 int8, fetched
// by direct global->LDS loads as two blocks of 8 whole 128-byte rows with the
// XOR-swizzled chunk order of the cooperative bf16 tiles (lane i: row i / 8,
// chunk (i % 8) ^ (i / 8) ^ 4 h), so the MFMA reads are conflict-free and
// every fetched line is used whole. The tile's block scales are staged once
// into LDS as f32 [block][row] (weights) and [block][token] (activations).
// Per block: one int8 MFMA 16x16x32 gives the exact integer block dot, then
// acc += float(isum) * (d_w * d_x) -- the same expression, in the same block
// order, as gemm_q8_kernel, so both produce the same bits. With p.splits > 1
// the grid also runs over K slices, each summing its blocks in order into
// its own f32 partial (the consumer adds the slices).
namespace {
typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void q8_g2l16(const void *src, void *lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t *) lds_base, 16, 0, 0);
}
template <int N>
__device__ __forceinline__ void q8_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
}  // namespace

// One output tile of problem p; li = the workgroup's index within p's tiles
// (p is a kernel argument read by name, never through a runtime index)
template <int TM, int TN, int R, int EPI, bool YBF16>
__device__ __forceinline__ void q8c_tile(const GemmParams &p, const int li, const int tiles_m, const int tiles_n) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int BM = 16 * TM, BN = 16 * TN, TMW = TM / 2, TNW = TN / 2;
    constexpr int U = TM + TN, USZ = 2048, STG = U * USZ, LW = 2 * U / 4;
    static_assert(TM % 2 == 0 && TN % 2 == 0 && (2 * U) % 4 == 0 && R >= 2 && R <= 4, "tile shape");
    // (m tile, K slice) units c = tm * S + sp; K slice sp covers blocks
    // [kbase, kbase + KB) of rows KBR blocks long
    const int S = p.splits > 1 ? p.splits : 1;
    const int KBR = p.K / 32, KB = KBR / S, ns = KB / 4;
    const int cm = tiles_m * S;
    int c, tn;
    if ((cm & 7) == 0) {
        // XCD x (= workgroup id mod 8) owns units x, x + 8, ... and every token tile of each
        const int sidx = li >> 3;
        c = (li & 7) + 8 * (sidx / tiles_n);
        tn = sidx % tiles_n;
    } else {
        c = li % cm;
        tn = li / cm;
    }
    if (c >= cm || tn >= tiles_n) return;
    const int tm = c / S, sp = c - tm * S;
    const int kb0s = KB * sp;                       // first block of this slice
    const int bm0 = tm * BM, bn0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int lr = lane & 15, lg = lane >> 4;

    // block scales of one segment of up to SEG blocks, f32: dws[kb][row],
    // dxs[kb][token]. Lane = row (token): four blocks per load, LDS writes of
    // consecutive rows for one block (conflict-free). A segment's scales are
    // loaded into registers during the last stage of the previous segment and
    // written to LDS at the next segment's first stage, between two barriers.
    constexpr int SEG = Q8_SEG, PW = (SEG / 4 * BM + 255) / 256, PX = (SEG / 4 * BN + 255) / 256;
    constexpr int SPS = SEG / 4;                       // stages per segment
    float *dws = (float *) (lds + R * STG);
    float *dxs = dws + min(KB, SEG) * BM;
    u32x2 pw[PW];
    f32x4 px[PX];
    auto load_scales = [&](int seg) {
        const int kb0 = seg * SEG, nq = min(KB - kb0, SEG) / 4;
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int e = tid + 256 * i, row = e % BM, q4 = e / BM;
            if (q4 < nq) pw[i] = *(const u32x2 *) (p.dw + (int64_t) min(bm0 + row, p.M - 1) * KBR + kb0s + kb0 + 4 * q4);
        }
#pragma unroll
        for (int i = 0; i < PX; ++i) {
            const int e = tid + 256 * i, tok = e % BN, q4 = e / BN;
            if (q4 < nq) px[i] = *(const f32x4 *) (p.dx + (int64_t) min(bn0 + tok, p.N - 1) * KBR + kb0s + kb0 + 4 * q4);
        }
    };
    auto store_scales = [&](int seg) {
        const int nq = min(KB - seg * SEG, SEG) / 4;
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int e = tid + 256 * i, row = e % BM, q4 = e / BM;
            const uint16_t *h = (const uint16_t *) &pw[i];
            if (q4 < nq)
#pragma unroll
                for (int c = 0; c < 4; ++c) dws[(4 * q4 + c) * BM + row] = f16_bits_to_f32(h[c]);
        }
#pragma unroll
        for (int i = 0; i < PX; ++i) {
            const int e = tid + 256 * i, tok = e % BN, q4 = e / BN;
            if (q4 < nq)
#pragma unroll
                for (int c = 0; c < 4; ++c) dxs[(4 * q4 + c) * BN + tok] = px[i][c];
        }
    };
    load_scales(0);
    store_scales(0);
    __syncthreads();

    // this wave's loads: fragment f = wave + 4 q is unit f / 2 (A units first), half f % 2
    const int r8 = lane >> 3;
    const int8_t *qsrc[LW];
    int qlds[LW];
#pragma unroll
    for (int q = 0; q < LW; ++q) {
        const int f = wave + 4 * q, u = f >> 1, h = f & 1;
        const int chunk = ((lane & 7) ^ r8 ^ (4 * h)) * 16;
        qlds[q] = u * USZ + h * 1024;
        if (u < TM) {
            const int rb = min((bm0 >> 4) + u, (p.M >> 4) - 1);
            qsrc[q] = p.qw + (int64_t) (rb * 16 + 8 * h + r8) * p.K + 32 * kb0s + chunk;
        } else {
            const int n = min(bn0 + 16 * (u - TM) + 8 * h + r8, p.N - 1);
            qsrc[q] = p.qx + (int64_t) n * p.K + 32 * kb0s + chunk;
        }
    }
    auto issue = [&](int t, int slot) {
        uint8_t *dst = lds + slot * STG;
#pragma unroll
        for (int q = 0; q < LW; ++q) q8_g2l16(qsrc[q] + (int64_t) t * 128, dst + qlds[q]);
    };
    // MFMA operand read offsets: row t = lane % 16, bytes 32 b + 8 (lane / 16) of the row
    int roff[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const int c = 2 * b + (lg >> 1);
        roff[b] = (lr >> 3) * 1024 + (lr & 7) * 128 + ((c ^ (lr & 7) ^ (4 * (lr >> 3))) * 16) + (lg & 1) * 8;
    }

    f32x4 acc[TMW][TNW];
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

#pragma unroll
    for (int st = 0; st < R - 1; ++st)
        if (st < ns) issue(st, st);
    int slot = 0;
    for (int t = 0; t < ns; ++t) {
        // own loads of stage t landed (at most min(ns - 1 - t, R - 2) later stages in flight)
        const int rem = min(ns - 1 - t, R - 2);
        const bool seg_start = t > 0 && t % SPS == 0;
        if (seg_start) {
            q8_wait_vm<0>();                     // the segment's scale loads are the youngest
        } else if constexpr (R >= 4) {
            if (rem >= 2) q8_wait_vm<2 * LW>();
            else if (rem == 1) q8_wait_vm<LW>();
            else q8_wait_vm<0>();
        } else if constexpr (R == 3) {
            if (rem >= 1) q8_wait_vm<LW>();
            else q8_wait_vm<0>();
        } else {
            q8_wait_vm<0>();
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (seg_start) {
            // every wave's reads of the previous segment's scales are done
            store_scales(t / SPS);
            __syncthreads();
        }
        if (t + R - 1 < ns) issue(t + R - 1, slot == 0 ? R - 1 : slot - 1);
        if (t % SPS == SPS - 1 && t + 1 < ns) load_scales(t / SPS + 1);
        const uint8_t *src = lds + slot * STG;
        // all block MFMAs of the stage first (independent results), then the
        // rescales in block order, so no MFMA waits on the previous one's read-out
        i32x4 isum[4][TMW][TNW];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            long a[TMW], bq[TNW];
#pragma unroll
            for (int i = 0; i < TMW; ++i) a[i] = *(const long *) (src + (wm * TMW + i) * USZ + roff[b]);
#pragma unroll
            for (int j = 0; j < TNW; ++j) bq[j] = *(const long *) (src + (TM + wn * TNW + j) * USZ + roff[b]);
#pragma unroll
            for (int i = 0; i < TMW; ++i)
#pragma unroll
                for (int j = 0; j < TNW; ++j)
                    isum[b][i][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], bq[j], i32x4{0, 0, 0, 0}, 0, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int kb = 4 * (t % SPS) + b;
            f32x4 dwv[TMW];
            float dxv[TNW];
#pragma unroll
            for (int i = 0; i < TMW; ++i) dwv[i] = *(const f32x4 *) &dws[kb * BM + 16 * (wm * TMW + i) + 4 * lg];
#pragma unroll
            for (int j = 0; j < TNW; ++j) dxv[j] = dxs[kb * BN + 16 * (wn * TNW + j) + lr];
#pragma unroll
            for (int i = 0; i < TMW; ++i)
#pragma unroll
                for (int j = 0; j < TNW; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][j][r] += (float) isum[b][i][j][r] * (dwv[i][r] * dxv[j]);
        }
        slot = slot + 1 == R ? 0 : slot + 1;
    }

    int m0[TMW], nn[TNW];
#pragma unroll
    for (int i = 0; i < TMW; ++i) m0[i] = bm0 + 16 * (wm * TMW + i) + 4 * lg;
#pragma unroll
    for (int j = 0; j < TNW; ++j) nn[j] = bn0 + 16 * (wn * TNW + j) + lr;
    if constexpr (EPI == EPI_GELU_Q8) {
        // GELU, then ggml's Q8_0 conversion of every token's 32-feature block
        // (the arithmetic of quantize_rows_q8_kernel: the same bits as storing
        // the f32 GELU rows and quantizing them). A block is this wave's 32
        // rows (TMW = 2), or 16 rows in each of the waves wm = 0, 1 (TMW = 1:
        // partial maxima exchanged through LDS). Lanes lg = 0..3 hold rows
        // 4 lg .. 4 lg + 3 of a 16-row fragment for token lr.
        float v[TMW][TNW][4], am[TNW];
#pragma unroll
        for (int j = 0; j < TNW; ++j) am[j] = 0.0f;
#pragma unroll
        for (int i = 0; i < TMW; ++i) {
            float bv[4] = {0.f, 0.f, 0.f, 0.f};
            if (p.bias && m0[i] < p.M)
                for (int r = 0; r < 4; ++r) bv[r] = p.bias[m0[i] + r];
#pragma unroll
            for (int j = 0; j < TNW; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    v[i][j][r] = gelu_tanh_f(acc[i][j][r] + bv[r]);
                    am[j] = fmaxf(am[j], fabsf(v[i][j][r]));
                }
        }
#pragma unroll
        for (int j = 0; j < TNW; ++j) {
            am[j] = fmaxf(am[j], __shfl_xor(am[j], 16));
            am[j] = fmaxf(am[j], __shfl_xor(am[j], 32));
        }
        if constexpr (TMW == 1) {
            float *xa = (float *) lds;
            __syncthreads();                     // every wave is done with the ring
#pragma unroll
            for (int j = 0; j < TNW; ++j)
                if (lg == 0) xa[((wn * TNW + j) * 16 + lr) * 2 + wm] = am[j];
            __syncthreads();
#pragma unroll
            for (int j = 0; j < TNW; ++j) {
                const int e = ((wn * TNW + j) * 16 + lr) * 2;
                am[j] = fmaxf(xa[e], xa[e + 1]);
            }
        }
        const int kb = (bm0 >> 5) + (TMW == 2 ? wm : 0);
#pragma unroll
        for (int j = 0; j < TNW; ++j) {
            const int n = nn[j];
            if (n >= p.N || bm0 >= p.M) continue;
            const float d = am[j] / 127.0f;
            const float id = am[j] != 0.0f ? 127.0f / am[j] : 0.0f;
            if (lg == 0 && (TMW == 2 || wm == 0)) p.yd[(int64_t) n * (p.M / 32) + kb] = f16_bits_to_f32(f32_to_f16_bits(d));
#pragma unroll
            for (int i = 0; i < TMW; ++i) {
                int8_t q[4];
                for (int r = 0; r < 4; ++r) q[r] = (int8_t) __builtin_rintf(v[i][j][r] * id);
                uint32_t w4;
                __builtin_memcpy(&w4, q, 4);
                *(uint32_t *) ((int8_t *) p.y + (int64_t) n * p.ld_y + m0[i]) = w4;
            }
        }
    } else if constexpr (EPI == EPI_QKV_ATTN) {
        // acc + bias staged token-major in LDS, then one wave per token: lane d
        // runs launch_qkv_scatter's arithmetic on feature d of the tile's head
        // (the same operations in the same order as storing the f32 rows and
        // scattering them, so the same bits)
        static_assert(BM == 64, "a tile is one head's q, k or v");
        constexpr int LDT = BM + 1;
        float *tt = (float *) lds;
        float bv[TMW][4];
#pragma unroll
        for (int i = 0; i < TMW; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) bv[i][r] = p.bias ? p.bias[m0[i] + r] : 0.0f;
        __syncthreads();                         // every wave is done with the ring
#pragma unroll
        for (int i = 0; i < TMW; ++i)
#pragma unroll
            for (int j = 0; j < TNW; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) tt[(nn[j] - bn0) * LDT + (m0[i] - bm0) + r] = acc[i][j][r] + bv[i][r];
        __syncthreads();
        // row (lane / 16) of wave w: tokens 4 (w + 4 i) + lane / 16, features
        // 4 sl .. 4 sl + 3 (tokens past N repeat token N - 1, same stores)
        const int H = p.qs.nh * 64, sec = bm0 / H, head = (bm0 - sec * H) >> 6, sl = lane & 15;
        for (int t0 = 4 * wave; t0 < BN; t0 += 16) {
            if (bn0 + t0 >= p.N) break;
            const int t = min(t0 + (lane >> 4), p.N - 1 - bn0);
            const float *src = tt + t * LDT + 4 * sl;
            const float x[4] = {src[0], src[1], src[2], src[3]};
            qkv_row_store(p.qs, sec, head, bn0 + t, x, sl);
        }
    } else if (S > 1) {
        // this slice's partial sums, no bias (the host allows EPI_STORE into f32 only)
        GemmParams q = p;
        q.y = (float *) p.y + sp * p.part_stride;
        q.bias = nullptr;
        epilogue_frags<EPI, YBF16, TMW, TNW>(q, m0, nn, acc);
    } else {
        epilogue_frags<EPI, YBF16, TMW, TNW>(p, m0, nn, acc);
    }
}

template <int TM, int TN, int R, int EPI, bool YBF16>
__global__ __launch_bounds__(256) void gemm_q8c_kernel(const GemmParams p, int tiles_m, int tiles_n) {
    q8c_tile<TM, TN, R, EPI, YBF16>(p, (int) blockIdx.x, tiles_m, tiles_n);
}

// two problems in one launch (the latent and text streams of a joint block):
// workgroups from begin1 (a multiple of 8, so that the XCD a unit lands on is
// the same in both numberings) run p1
template <int TM, int TN, int R, int EPI, bool YBF16>
__global__ __launch_bounds__(256) void gemm_q8c_pair_kernel(const GemmParams p0, const GemmParams p1, int tm0, int tn0,
                                                            int tm1, int tn1, int begin1) {
    if ((int) blockIdx.x >= begin1) q8c_tile<TM, TN, R, EPI, YBF16>(p1, (int) blockIdx.x - begin1, tm1, tn1);
    else q8c_tile<TM, TN, R, EPI, YBF16>(p0, (int) blockIdx.x, tm0, tn0);
}

// ------------------------------------------------------------------ activation quantization
// One thread per 32-block: d = amax/127 (stored as the fp32 value of its fp16
// rounding), q = rne(x * (127/amax)) — ggml-cpu's x86 quantize_row_q8_0.
// Row n of the output reads source row (n / grp) * gstride + n % grp (grp
// > 0: rows gathered from a grouped layout, e.g. one stream's tokens of every
// batch item in [B][Ntot] rows), else row n.
// one 32-element block blk of rows from x (see quantize_rows_q8_kernel)
template <bool XF32>
__device__ __forceinline__ void quantize_block_q8(const void *x, int64_t ld_x, int K, int8_t *qx, float *dx, int grp,
                                                  int64_t gstride, const int64_t blk) {
    const int KB = K / 32;
    const int row = (int) (blk / KB), kb = (int) (blk % KB);
    const int64_t src = grp > 0 ? (int64_t) (row / grp) * gstride + row % grp : row;
    float v[32];
    if constexpr (XF32) {
        const float *xr = (const float *) x + src * ld_x + kb * 32;
        for (int j = 0; j < 32; j += 4) {
            f32x4 t = *(const f32x4 *) (xr + j);
            v[j] = t[0]; v[j + 1] = t[1]; v[j + 2] = t[2]; v[j + 3] = t[3];
        }
    } else {
        const uint16_t *xr = (const uint16_t *) x + src * ld_x + kb * 32;
        for (int j = 0; j < 32; ++j) v[j] = bf16_bits_to_f32(xr[j]);
    }
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
    const float d = amax / 127.0f;
    const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
    dx[(int64_t) row * KB + kb] = f16_bits_to_f32(f32_to_f16_bits(d));
    int8_t q[32];
    for (int j = 0; j < 32; ++j) q[j] = (int8_t) __builtin_rintf(v[j] * id);
    int8_t *o = qx + (int64_t) row * K + kb * 32;
    *(u32x4 *) o = *(const u32x4 *) q;
    *(u32x4 *) (o + 16) = *(const u32x4 *) (q + 16);
}

template <bool XF32>
__global__ void quantize_rows_q8_kernel(const void *x, int64_t ld_x, int N, int K, int8_t *qx, float *dx, int grp,
                                        int64_t gstride) {
    const int64_t blk = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (blk < (int64_t) N * (K / 32)) quantize_block_q8<XF32>(x, ld_x, K, qx, dx, grp, gstride, blk);
}

// two row sets (two streams) in one launch: blocks from N0 * K / 32 on quantize set 1
__global__ void quantize_rows_q8_pair_kernel(const QuantRows r0, const QuantRows r1) {
    const int64_t blk = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n0 = (int64_t) r0.N * (r0.K / 32);
    if (blk < n0) quantize_block_q8<true>(r0.x, r0.ld_x, r0.K, r0.qx, r0.dx, r0.grp, r0.gstride, blk);
    else if (blk - n0 < (int64_t) r1.N * (r1.K / 32))
        quantize_block_q8<true>(r1.x, r1.ld_x, r1.K, r1.qx, r1.dx, r1.grp, r1.gstride, blk - n0);
}

// ------------------------------------------------------------------ dispatch
template <int WM, int WN, int TM, int TN, bool XF32, bool YBF16>
hipError_t gemm_bf16_epi(const GemmParams &p, hipStream_t s) {
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    dim3 grid((p.M + BM - 1) / BM, (p.N + BN - 1) / BN);
    dim3 block(WM * WN * 64);
    switch (p.epi) {
        case EPI_GELU:
            launch_kernel((gemm_bf16_kernel<WM, WN, TM, TN, XF32, EPI_GELU, YBF16>), grid, block, 0, s, p);
            break;
        case EPI_GATE_RES:
            launch_kernel((gemm_bf16_kernel<WM, WN, TM, TN, XF32, EPI_GATE_RES, false>), grid, block, 0, s, p);
            break;
        default:
            launch_kernel((gemm_bf16_kernel<WM, WN, TM, TN, XF32, EPI_STORE, YBF16>), grid, block, 0, s, p);
    }
    return hipGetLastError();
}


template <int WM, int WN, int TM, int TN, bool YBF16>
hipError_t gemm_q8_epi(const GemmParams &p, hipStream_t s) {
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    dim3 grid((p.M + BM - 1) / BM, (p.N + BN - 1) / BN);
    dim3 block(WM * WN * 64);
    switch (p.epi) {
        case EPI_GELU:
            launch_kernel((gemm_q8_kernel<WM, WN, TM, TN, EPI_GELU, YBF16>), grid, block, 0, s, p);
            break;
        case EPI_GATE_RES:
            launch_kernel((gemm_q8_kernel<WM, WN, TM, TN, EPI_GATE_RES, false>), grid, block, 0, s, p);
            break;
        case EPI_GEGLU:
            if (p.M % 4 || p.y_bf16) return hipErrorInvalidValue;
            launch_kernel((gemm_q8_kernel<WM, WN, TM, TN, EPI_GEGLU, false>), grid, block, 0, s, p);
            break;
        default:
            launch_kernel((gemm_q8_kernel<WM, WN, TM, TN, EPI_STORE, YBF16>), grid, block, 0, s, p);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_bf16(const GemmParams &p, hipStream_t s) {
    if (p.epi != EPI_STORE) return hipErrorInvalidValue;
    GemmGroup g;
    memset(&g, 0, sizeof(g));
    g.nprob = 1;
    GemmProblem &q = g.p[0];
    q.x = p.x; q.w = (const uint16_t *) p.w; q.bias = p.bias; q.y = p.y;
    q.ld_x = p.ld_x; q.ld_w = p.ld_w; q.ld_y = p.ld_y;
    q.x_group_rows = p.x_group_rows; q.x_group_stride = p.x_group_stride;
    q.M = p.M; q.N = p.N; q.K = p.K; q.splits = 1;
    return launch_gemm_group(g, p.x_f32 ? GEMM_X_F32 : 0, p.y_bf16 ? EPI_STORE_BF16 : EPI_STORE_F32, s);
}

namespace {

template <int TM, int TN, int R, int EPI, bool YBF16>
hipError_t q8c_launch(const GemmParams &p, hipStream_t s) {
    constexpr int BM = 16 * TM, BN = 16 * TN;
    const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
    const size_t lds = (size_t) R * (TM + TN) * 2048 + (size_t) std::min(p.K / 32, Q8_SEG) * (BM + BN) * 4;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    auto kern = gemm_q8c_kernel<TM, TN, R, EPI, YBF16>;
    lds_opt_in((const void *) kern, lds);
    launch_kernel(kern, dim3(tiles_m * tiles_n * (p.splits > 1 ? p.splits : 1)), dim3(256), lds, s, p, tiles_m,
                  tiles_n);
    return hipGetLastError();
}

template <int TM, int TN, int R, int EPI, bool YBF16>
hipError_t q8c_launch_pair(const GemmParams &p0, const GemmParams &p1, hipStream_t s) {
    constexpr int BM = 16 * TM, BN = 16 * TN;
    const int tm0 = (p0.M + BM - 1) / BM, tn0 = (p0.N + BN - 1) / BN;
    const int tm1 = (p1.M + BM - 1) / BM, tn1 = (p1.N + BN - 1) / BN;
    const int S0 = p0.splits > 1 ? p0.splits : 1, S1 = p1.splits > 1 ? p1.splits : 1;
    const size_t lds = (size_t) R * (TM + TN) * 2048 +
                       (size_t) std::min(std::max(p0.K, p1.K) / 32, Q8_SEG) * (BM + BN) * 4;
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    auto kern = gemm_q8c_pair_kernel<TM, TN, R, EPI, YBF16>;
    lds_opt_in((const void *) kern, lds);
    const int begin1 = (tm0 * tn0 * S0 + 7) & ~7;
    launch_kernel(kern, dim3(begin1 + tm1 * tn1 * S1), dim3(256), lds, s, p0, p1, tm0, tn0, tm1, tn1, begin1);
    return hipGetLastError();
}

template <int TM, int TN, int R, bool YBF16>
hipError_t q8c_epi_pair(const GemmParams &p0, const GemmParams &p1, hipStream_t s) {
    switch (p0.epi) {
        case EPI_GELU: return q8c_launch_pair<TM, TN, R, EPI_GELU, YBF16>(p0, p1, s);
        case EPI_GATE_RES: return q8c_launch_pair<TM, TN, R, EPI_GATE_RES, false>(p0, p1, s);
        case EPI_GELU_Q8: return q8c_launch_pair<TM, TN, R, EPI_GELU_Q8, false>(p0, p1, s);
        case EPI_QKV_ATTN:
            if constexpr (TM == 4) return q8c_launch_pair<TM, TN, R, EPI_QKV_ATTN, false>(p0, p1, s);
            else return hipErrorInvalidValue;
        case EPI_STORE: return q8c_launch_pair<TM, TN, R, EPI_STORE, YBF16>(p0, p1, s);
        default: return hipErrorInvalidValue;
    }
}

template <int TM, int TN, int R, bool YBF16>
hipError_t q8c_epi(const GemmParams &p, hipStream_t s) {
    switch (p.epi) {
        case EPI_GELU: return q8c_launch<TM, TN, R, EPI_GELU, YBF16>(p, s);
        case EPI_GATE_RES: return q8c_launch<TM, TN, R, EPI_GATE_RES, false>(p, s);
        case EPI_GEGLU:
            if (p.M % 4 || p.y_bf16) return hipErrorInvalidValue;
            return q8c_launch<TM, TN, R, EPI_GEGLU, false>(p, s);
        case EPI_GELU_Q8: return q8c_launch<TM, TN, R, EPI_GELU_Q8, false>(p, s);
        case EPI_QKV_ATTN:
            if constexpr (TM == 4) return q8c_launch<TM, TN, R, EPI_QKV_ATTN, false>(p, s);
            else return hipErrorInvalidValue;
        default: return q8c_launch<TM, TN, R, EPI_STORE, YBF16>(p, s);
    }
}

}  // namespace

// EPI_QKV_ATTN: the attention operands of one stream (3 nh heads of 64
// rows, every pointer the scatter writes or reads)
static bool qkv_attn_ok(const GemmParams &p) {
    const QkvScatter &q = p.qs;
    return p.splits <= 1 && !p.y_bf16 && q.nh > 0 && p.M == 3 * 64 * q.nh && q.seq > 0 && p.N % q.seq == 0 && q.q &&
           q.k && q.vt && q.qn_w && q.kn_w && (!q.rope || q.rope_cs) && q.ldv % 16 == 0 && q.ldv >= q.Ntot &&
           q.Ntot >= q.tok_off + q.seq && q.tok_off >= 0;
}

hipError_t launch_gemm_q8(const GemmParams &p, hipStream_t s) {
    // cooperative tiles when the planes allow them: K % 128 (four-block
    // stages), M % 16, 16-byte aligned rows; block scales staged in segments
    // of 1024 k (three 64 x 64 workgroups per CU). Measured on MI355X at 1446
    // rows: 64 x 64 tiles with a 2-stage ring (1024 -> 3072: 51.5 -> 34.7 us
    // against the 2 x 2-wave kernel below, which stays for other shapes;
    // Tuning::q8_old forces it for comparisons).
    const Tuning &tu = tuning();
    const int S = p.splits > 1 ? p.splits : 1;
    const bool coop = p.K % (128 * S) == 0 && p.M % 16 == 0 && ((uintptr_t) p.qw & 15) == 0 &&
                      ((uintptr_t) p.qx & 15) == 0 && ((uintptr_t) p.dw & 7) == 0 && ((uintptr_t) p.dx & 15) == 0 &&
                      !tu.q8_old;
    // split-K partials: cooperative tiles only, f32 stores of the slices
    if (S > 1 && (!coop || p.epi != EPI_STORE || p.y_bf16 || p.part_stride < (int64_t) p.N * p.ld_y))
        return hipErrorInvalidValue;
    // GELU into Q8_0 planes: cooperative tiles only, whole 32-feature blocks
    // in every tile
    if (p.epi == EPI_GELU_Q8 && (!coop || S > 1 || p.y_bf16 || p.M % 64 || !p.yd || p.ld_y < p.M || p.ld_y % 4))
        return hipErrorInvalidValue;
    // the attention operands: 64 x 64 tiles only (a tile is one head)
    if (p.epi == EPI_QKV_ATTN)
        return coop && qkv_attn_ok(p) ? q8c_epi<4, 4, 2, false>(p, s) : hipErrorInvalidValue;
    if (coop) {
        // 64 x 64 tiles with a 2-stage ring; 32 x 64 (weight rows x tokens)
        // when the 64 x 64 grid would hold fewer than two tiles per CU
        // (measured: 1446 x 1024 outputs at K = 1024 / 4096 19.8 -> 18.1 / 54.4
        // -> 48.3 us; the T5 o / wo projections). Tuning::q8_cfg picks a
        // shape: 2 = 64 x 64 / 2 stages, 5 = 32 x 64 (2 stages); sweep builds
        // (TSK_SWEEP_VARIANTS) add 1 = 64 x 64 / 3 stages, 3 = 128 x 64,
        // 4 = 64 x 128
        const int64_t tiles64 = (int64_t) ((p.M + 63) / 64) * ((p.N + 63) / 64);
        const int cfg = tu.q8_cfg ? tu.q8_cfg : tiles64 * S < 512 ? 5 : 2;
        switch (cfg) {
            case 2: return p.y_bf16 ? q8c_epi<4, 4, 2, true>(p, s) : q8c_epi<4, 4, 2, false>(p, s);
            case 5: return p.y_bf16 ? q8c_epi<2, 4, 2, true>(p, s) : q8c_epi<2, 4, 2, false>(p, s);
#if TSK_SWEEP_VARIANTS
            case 1: return p.y_bf16 ? q8c_epi<4, 4, 3, true>(p, s) : q8c_epi<4, 4, 3, false>(p, s);
            case 3: return p.y_bf16 ? q8c_epi<8, 4, 2, true>(p, s) : q8c_epi<8, 4, 2, false>(p, s);
            case 4: return p.y_bf16 ? q8c_epi<4, 8, 2, true>(p, s) : q8c_epi<4, 8, 2, false>(p, s);
#endif
            default: return hipErrorInvalidValue;
        }
    }
    return p.y_bf16 ? gemm_q8_epi<2, 2, 2, 2, true>(p, s) : gemm_q8_epi<2, 2, 2, 2, false>(p, s);
}

hipError_t launch_gemm_q8_pair(const GemmParams &p0, const GemmParams &p1, hipStream_t s) {
    // one launch when both problems take the cooperative tiles with the same
    // epilogue, output type and split count (each output is still summed in
    // the same order, whatever the tile shape or the launch it runs in);
    // otherwise two launches
    const Tuning &tu = tuning();
    auto coop = [&](const GemmParams &p) {
        const int S = p.splits > 1 ? p.splits : 1;
        return p.K % (128 * S) == 0 && p.M % 16 == 0 && ((uintptr_t) p.qw & 15) == 0 && ((uintptr_t) p.qx & 15) == 0 &&
               ((uintptr_t) p.dw & 7) == 0 && ((uintptr_t) p.dx & 15) == 0 && !tu.q8_old;
    };
    const bool pair = tu.q8_pair && coop(p0) && coop(p1) && p0.epi == p1.epi && p0.y_bf16 == p1.y_bf16 &&
                      p0.splits == p1.splits && p0.epi != EPI_GEGLU;
    if (pair) {
        const int S = p0.splits > 1 ? p0.splits : 1;
        // the single-problem checks of launch_gemm_q8, on each problem
        for (const GemmParams *p : {&p0, &p1}) {
            if (S > 1 && (p->epi != EPI_STORE || p->y_bf16 || p->part_stride < (int64_t) p->N * p->ld_y))
                return hipErrorInvalidValue;
            if (p->epi == EPI_GELU_Q8 && (S > 1 || p->y_bf16 || p->M % 64 || !p->yd || p->ld_y < p->M || p->ld_y % 4))
                return hipErrorInvalidValue;
            if (p->epi == EPI_QKV_ATTN && !qkv_attn_ok(*p)) return hipErrorInvalidValue;
        }
        if (p0.epi == EPI_QKV_ATTN) return q8c_epi_pair<4, 4, 2, false>(p0, p1, s);
        const int64_t tiles64 = (int64_t) ((p0.M + 63) / 64) * ((p0.N + 63) / 64) +
                                (int64_t) ((p1.M + 63) / 64) * ((p1.N + 63) / 64);
        const int cfg = tu.q8_cfg ? tu.q8_cfg : tiles64 * S < 512 ? 5 : 2;
        if (cfg == 2) return p0.y_bf16 ? q8c_epi_pair<4, 4, 2, true>(p0, p1, s) : q8c_epi_pair<4, 4, 2, false>(p0, p1, s);
        if (cfg == 5) return p0.y_bf16 ? q8c_epi_pair<2, 4, 2, true>(p0, p1, s) : q8c_epi_pair<2, 4, 2, false>(p0, p1, s);
    }
    hipError_t e = launch_gemm_q8(p0, s);
    return e != hipSuccess ? e : launch_gemm_q8(p1, s);
}

hipError_t launch_quantize_rows_q8_pair(const QuantRows &r0, const QuantRows &r1, hipStream_t s) {
    for (const QuantRows *r : {&r0, &r1})
        if (r->N < 1 || r->K < 32 || r->K % 32) return hipErrorInvalidValue;
    const int64_t nblk = (int64_t) r0.N * (r0.K / 32) + (int64_t) r1.N * (r1.K / 32);
    launch_kernel(quantize_rows_q8_pair_kernel, dim3((unsigned) ((nblk + 255) / 256)), dim3(256), 0, s, r0, r1);
    return hipGetLastError();
}

hipError_t launch_quantize_rows_q8(const void *x, int x_f32, int64_t ld_x, int N, int K, int8_t *qx, float *dx,
                                   hipStream_t s, int grp, int64_t gstride) {
    const int64_t nblk = (int64_t) N * (K / 32);
    const int threads = 256;
    dim3 grid((unsigned) ((nblk + threads - 1) / threads));
    if (x_f32) launch_kernel(quantize_rows_q8_kernel<true>, grid, dim3(threads), 0, s, x, ld_x, N, K, qx, dx, grp, gstride);
    else launch_kernel(quantize_rows_q8_kernel<false>, grid, dim3(threads), 0, s, x, ld_x, N, K, qx, dx, grp, gstride);
    return hipGetLastError();
}

}  // namespace tsk
