// gemm_f32.hip — F32-weight GEMMs on gfx950: ggml_mul_mat with an F32 src0,
// whose vec_dot type is F32, so activations stay fp32 and every product and
// sum is fp32 (src/mmdit.cpp:13, :24 — the Q8_0 DiT keeps its 3-D
// convolution kernels in F32).
//
//   Y[n, m] = sum_k X[n, k] * W[m, k] + bias[m]
//
// fp32 MFMA 16x16x4: A = 16 weight rows, B = 16 tokens; lane l supplies row /
// token l % 16 at k-lane l / 16 and ends with 4 consecutive output features
// of one token. A 16-B LDS read gives each lane four k values
// (4 * (l / 16) + t, t = 0..3), consumed by four MFMAs, so one K block of 16
// costs TM + TN LDS reads for 4 * TM * TN MFMAs.
//
// Workgroup = 2 x 2 waves, each TM x TN 16x16 tiles (4 x 4 or 4 x 2, by the
// launcher's rule below); operand tiles are double buffered through LDS
// (global -> registers -> LDS, one barrier per 32-wide K step). The
// activation rows may be an implicit im2col of a channels-fastest input
// (GemmProblem::conv_ic, as in gemm_group.hip).
#include "tsk_common.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

namespace tsk {

namespace {

constexpr int NT = 256;
constexpr int BK = 32;
constexpr int LDK = BK + 4;   // floats per LDS row: 16-B aligned, the 16 rows of a read hit distinct banks

// The epilogue of both F32 kernels, through LDS: the accumulators as the
// workgroup's [BN][BM] tile (row stride LDT, in `tile`, free LDS of at least
// BN * LDT floats), then four consecutive outputs of one token per thread,
// BM / 4 threads a token row: whole-row stores of y / y2, and the SnakeBeta's
// sinf with one group of values live at a time
template <int TM, int TN, bool YBF16, bool SNAKE>
__device__ __forceinline__ void f32_epilogue(const GemmProblem &p, const F32Snake &sk, const f32x4 (&acc)[TM][TN],
                                             float *tile, int bm0, int bn0, int z) {
    constexpr int BM = 2 * TM * 16, BN = 2 * TN * 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int wm = wave & 1, wn = wave >> 1;
    constexpr int LDT = BM + 4;
    for (int i = 0; i < TM; ++i)
        for (int j = 0; j < TN; ++j)
            *(f32x4 *) &tile[((wn * TN + j) * 16 + lr) * LDT + (wm * TM + i) * 16 + 4 * lg] = acc[i][j];
    __syncthreads();
    // NT is a multiple of BM / 4: a thread keeps one group of four output
    // channels (its bias and SnakeBeta factors loaded once) over NT / (BM / 4)
    // token rows apart
    constexpr int G = BM / 4;
    static_assert(NT % G == 0, "fixed channel group per thread");
    const int ml = (tid % G) * 4, m0 = bm0 + ml;
    if (m0 >= p.M) return;
    const bool full = m0 + 3 < p.M;
    float bv[4], ea[4], eb[4];
    for (int r = 0; r < 4; ++r) {
        const bool in = m0 + r < p.M;
        bv[r] = (p.bias && in) ? p.bias[m0 + r] : 0.0f;
        ea[r] = eb[r] = 0.0f;
        if constexpr (SNAKE) {
            const int c0 = m0 % sk.period;   // period is a multiple of 4: c0 + 3 < period
            if (in) {
                ea[r] = sk.ea[c0 + r];
                eb[r] = sk.eb[c0 + r];
            }
        }
    }
    for (int nl = tid / G; nl < BN; nl += NT / G) {
        const int n = bn0 + nl;
        if (n >= p.N) break;
        const f32x4 a4 = *(const f32x4 *) &tile[nl * LDT + ml];
        float o[4];
        for (int r = 0; r < 4; ++r) o[r] = a4[r] + bv[r];
        if constexpr (YBF16) {
            uint16_t *yr = (uint16_t *) p.y + (int64_t) n * p.ld_y + m0;
            for (int r = 0; r < 4 && m0 + r < p.M; ++r) yr[r] = f32_to_bf16_bits(o[r]);
        } else {
            float *yr = (float *) p.y + (int64_t) z * p.N * p.ld_y + (int64_t) n * p.ld_y + m0;
            float v[4];
            if (p.accumulate) {
                if (full) {
                    const f32x4 a = *(const f32x4 *) yr;
                    for (int r = 0; r < 4; ++r) v[r] = a[r] + o[r];
                } else {
                    for (int r = 0; r < 4; ++r) v[r] = m0 + r < p.M ? yr[r] + o[r] : 0.0f;
                }
            } else {
                for (int r = 0; r < 4; ++r) v[r] = o[r];
            }
            float sv[4];
            if constexpr (SNAKE)
                for (int r = 0; r < 4; ++r) {
                    const float sn = sinf(v[r] * ea[r]);
                    sv[r] = v[r] + (sn * sn) * eb[r];
                }
            // y: the snake in place (SNAKE without y2) or the plain value;
            // y2: the snake next to it
            const bool in_place = SNAKE && !sk.y2;
            float w[4];
            for (int r = 0; r < 4; ++r) w[r] = in_place ? sv[r] : v[r];
            if (full) {
                *(f32x4 *) yr = f32x4{w[0], w[1], w[2], w[3]};
            } else {
                for (int r = 0; r < 4 && m0 + r < p.M; ++r) yr[r] = w[r];
            }
            if constexpr (SNAKE) {
                if (sk.y2) {
                    float *y2r = sk.y2 + (int64_t) n * p.ld_y + m0;
                    if (full) {
                        *(f32x4 *) y2r = f32x4{sv[0], sv[1], sv[2], sv[3]};
                    } else {
                        for (int r = 0; r < 4 && m0 + r < p.M; ++r) y2r[r] = sv[r];
                    }
                }
            }
        }
    }
}

template <int TM, int TN, bool YBF16, bool SNAKE>
__global__ __launch_bounds__(NT) void gemm_f32_kernel(const GemmProblem p, const F32Snake sk) {
    constexpr int BM = 2 * TM * 16, BN = 2 * TN * 16;
    constexpr int WCH = BM * (BK / 4), XCH = BN * (BK / 4);   // 16-B chunks per tile
    constexpr int WPER = WCH / NT, XPER = XCH / NT;
    static_assert(WCH % NT == 0 && XCH % NT == 0, "tile chunks");
    // operand buffers Ws[2][BM * LDK] and Xs[2][BN * LDK]; after the K loop
    // the same LDS holds the workgroup's output tile for the epilogue
    __shared__ __attribute__((aligned(16))) float smem[2 * (BM + BN) * LDK];
    float (*Ws)[BM * LDK] = reinterpret_cast<float (*)[BM * LDK]>(smem);
    float (*Xs)[BN * LDK] = reinterpret_cast<float (*)[BN * LDK]>(smem + 2 * BM * LDK);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const int wm = wave & 1, wn = wave >> 1;
    const int bm0 = blockIdx.x * BM, bn0 = blockIdx.y * BN;
    const float *W = p.wf;
    const float *X = (const float *) p.x;

    // per-chunk source rows, fixed over K: weight row, and for X the row
    // offset (plain) or batch offset + first input position (convolution)
    int64_t xbase[XPER];
    int xiw0[XPER];
    bool xrow_ok[XPER];
    for (int i = 0; i < XPER; ++i) {
        const int c = tid + i * NT;
        const int n = bn0 + c / (BK / 4);
        xrow_ok[i] = n < p.N;
        const int nn = xrow_ok[i] ? n : 0;
        if (p.conv_ic) {
            const int b = nn / p.conv_ow, ow = nn - b * p.conv_ow;
            xbase[i] = (int64_t) b * p.x_group_stride;
            xiw0[i] = ow * p.conv_s - p.conv_p;
        } else {
            xbase[i] = p.x_group_rows ? (int64_t) (nn / p.x_group_rows) * p.x_group_stride +
                                            (int64_t) (nn % p.x_group_rows) * p.ld_x
                                      : (int64_t) nn * p.ld_x;
            xiw0[i] = 0;
        }
    }

    f32x4 wreg[WPER], xreg[XPER];
    // split-K: slice z sums the k tiles [z nk / S, (z + 1) nk / S) into its own
    // output slice (the caller sums the slices in order)
    const int nk_all = (p.K + BK - 1) / BK, S = p.splits > 1 ? p.splits : 1, z = (int) blockIdx.z;
    const int kt0 = z * nk_all / S, nk = (z + 1) * nk_all / S;
    auto gload = [&](int kt) {
        const int k0 = kt * BK;
        for (int i = 0; i < WPER; ++i) {
            const int c = tid + i * NT;
            const int row = bm0 + c / (BK / 4), k = k0 + (c % (BK / 4)) * 4;
            wreg[i] = f32x4{0, 0, 0, 0};
            if (row < p.M && k < p.K) wreg[i] = *(const f32x4 *) (W + (int64_t) row * p.ld_w + k);
        }
        for (int i = 0; i < XPER; ++i) {
            const int c = tid + i * NT;
            const int k = k0 + (c % (BK / 4)) * 4;
            bool ok = xrow_ok[i] && k < p.K;
            int64_t off = 0;
            if (p.conv_ic) {
                const int kw = k / p.conv_ic, ic = k - kw * p.conv_ic;
                const int iw = xiw0[i] + kw * p.conv_d;
                ok = ok && iw >= 0 && iw < p.conv_iw;
                off = xbase[i] + (int64_t) iw * p.ld_x + ic;
            } else {
                off = xbase[i] + k;
            }
            xreg[i] = f32x4{0, 0, 0, 0};
            if (ok) xreg[i] = *(const f32x4 *) (X + off);
        }
    };
    auto lstore = [&](int buf) {
        for (int i = 0; i < WPER; ++i) {
            const int c = tid + i * NT;
            *(f32x4 *) &Ws[buf][(c / (BK / 4)) * LDK + (c % (BK / 4)) * 4] = wreg[i];
        }
        for (int i = 0; i < XPER; ++i) {
            const int c = tid + i * NT;
            *(f32x4 *) &Xs[buf][(c / (BK / 4)) * LDK + (c % (BK / 4)) * 4] = xreg[i];
        }
    };

    f32x4 acc[TM][TN];
    for (int i = 0; i < TM; ++i)
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    gload(kt0);
    lstore(0);
    __syncthreads();
    for (int kt = kt0; kt < nk; ++kt) {
        const int buf = (kt - kt0) & 1;
        if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
        for (int kb = 0; kb < BK / 16; ++kb) {
            f32x4 a[TM], b[TN];
            for (int i = 0; i < TM; ++i)
                a[i] = *(const f32x4 *) &Ws[buf][((wm * TM + i) * 16 + lr) * LDK + 16 * kb + 4 * lg];
            for (int j = 0; j < TN; ++j)
                b[j] = *(const f32x4 *) &Xs[buf][((wn * TN + j) * 16 + lr) * LDK + 16 * kb + 4 * lg];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                for (int i = 0; i < TM; ++i)
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][t], b[j][t], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    static_assert(BN * (BM + 4) <= 2 * (BM + BN) * LDK, "output tile fits the operand buffers");
    f32_epilogue<TM, TN, YBF16, SNAKE>(p, sk, acc, smem, bm0, bn0, z);
}

typedef __attribute__((address_space(3))) void lds_void;

// The same product with direct global -> LDS loads (buffer_load ... lds) into
// an NS-stage ring of 32-wide K steps: no register staging, NS - 1 steps in
// flight. A stage holds the BM weight rows then the BN activation rows, 128
// bytes each; a row's 16-byte chunk c sits at slot c ^ ((row / 2) % 8), so the
// 16 rows of an MFMA operand read hit 16 distinct slots (two rows per 256
// bytes of banks). Wave-load j of a stage fills rows 8 j .. 8 j + 7: lane i
// loads the global chunk (i % 8) ^ (((8 j + i / 8) / 2) % 8) of row
// 8 j + i / 8. Rows past M / N and convolution taps outside the input read as
// zeros through the buffers' ranges (tap offsets are moved past the range).
// The MFMAs and their k order are those of gemm_f32_kernel: the same bits.
template <int TM, int TN, int NS, bool YBF16, bool SNAKE>
__global__ __launch_bounds__(NT) void gemm_f32_dl_kernel(const GemmProblem p, const F32Snake sk, uint32_t x_bytes) {
    constexpr int BM = 2 * TM * 16, BN = 2 * TN * 16;
    constexpr int ROWS = BM + BN, STAGE = ROWS * BK;          // floats per stage
    constexpr int NWL = ROWS / 8, WLW = NWL / 4;             // wave-loads per stage, per wave
    static_assert(NWL % 4 == 0 && BM % 8 == 0, "whole wave-loads per wave");
    constexpr int RING = NS * STAGE, EPI_F = BN * (BM + 4);
    __shared__ __attribute__((aligned(16))) float smem[RING > EPI_F ? RING : EPI_F];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lg = lane >> 4;
    const int wm = wave & 1, wn = wave >> 1;
    const int bm0 = blockIdx.x * BM, bn0 = blockIdx.y * BN;

    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        (void *) p.wf, (short) 0, (int) ((int64_t) p.M * p.ld_w * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void *) p.x, (short) 0, (int) x_bytes,
                                                                         0x00020000);
    constexpr uint32_t PAST = 0x80000000u;                   // beyond every range: reads zero
    // this lane's rows of its wave-loads: weight row offsets (bytes), or the
    // activation row's batch offset and first input position
    uint32_t rowoff[WLW];
    int iw0[WLW];
    bool isw[WLW], nok[WLW];
#pragma unroll
    for (int q = 0; q < WLW; ++q) {
        const int j = wave * WLW + q, R = 8 * j + (lane >> 3);
        const int c = (lane & 7) ^ ((R >> 1) & 7);
        isw[q] = j < BM / 8;                                 // wave-uniform: the descriptor stays scalar
        if (isw[q]) {
            rowoff[q] = (uint32_t) (((int64_t) (bm0 + R) * p.ld_w + 4 * c) * 4);
            iw0[q] = 0;
            nok[q] = true;
        } else {
            const int n = bn0 + R - BM;
            nok[q] = n < p.N;
            const int nn = nok[q] ? n : 0;
            if (p.conv_ic) {
                const int b = nn / p.conv_ow, ow = nn - b * p.conv_ow;
                rowoff[q] = (uint32_t) (((int64_t) b * p.x_group_stride + 4 * c) * 4);
                iw0[q] = ow * p.conv_s - p.conv_p;
            } else {
                rowoff[q] = (uint32_t) (((int64_t) nn * p.ld_x + 4 * c) * 4);
                iw0[q] = 0;
            }
        }
    }
    const int nk_all = p.K / BK, S = p.splits > 1 ? p.splits : 1, z = (int) blockIdx.z;
    const int kt0 = z * nk_all / S, nk = (z + 1) * nk_all / S;
    auto issue = [&](int kt, int slot) {
        const int k0 = kt * BK;
        float *st = smem + slot * STAGE;
        int kw = 0, ic0 = k0;
        if (p.conv_ic) {
            kw = k0 / p.conv_ic;
            ic0 = k0 - kw * p.conv_ic;
        }
#pragma unroll
        for (int q = 0; q < WLW; ++q) {
            const int j = wave * WLW + q;
            uint32_t off;
            if (isw[q]) {
                off = rowoff[q] + (uint32_t) (k0 * 4);
            } else if (p.conv_ic) {
                const int iw = iw0[q] + kw * p.conv_d;
                const bool ok = nok[q] && iw >= 0 && iw < p.conv_iw;
                off = ok ? rowoff[q] + (uint32_t) (((int64_t) iw * p.ld_x + ic0) * 4) : PAST;
            } else {
                off = nok[q] ? rowoff[q] + (uint32_t) (k0 * 4) : PAST;
            }
            // (a conditional expression choosing the descriptor leaves the
            // kernel uninstantiated on the host side: two calls instead)
            if (isw[q])
                __builtin_amdgcn_raw_ptr_buffer_load_lds(wrs, (lds_void *) (st + j * 8 * BK), 16, off, 0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (lds_void *) (st + j * 8 * BK), 16, off, 0, 0, 0);
        }
    };

    f32x4 acc[TM][TN];
    for (int i = 0; i < TM; ++i)
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0, 0, 0, 0};
    // LDS float offset of this lane's 16 bytes of operand row `row`, chunk c
    auto at = [](int row, int c) { return row * BK + ((c ^ ((row >> 1) & 7)) << 2); };

#pragma unroll
    for (int s0 = 0; s0 < NS - 1; ++s0)
        if (kt0 + s0 < nk) issue(kt0 + s0, s0);
    for (int kt = kt0; kt < nk; ++kt) {
        const int it = kt - kt0, slot = it % NS;
        // this wave's loads of step kt have landed once at most the later
        // steps' (up to NS - 2 of them) are outstanding; the barrier covers
        // the other waves' loads and frees the slot that step kt + NS - 1 fills
        if constexpr (NS == 3) {
            if (kt + 1 < nk) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WLW) : "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();
        if (kt + NS - 1 < nk) issue(kt + NS - 1, (it + NS - 1) % NS);
        const float *st = smem + slot * STAGE;
#pragma unroll
        for (int kb = 0; kb < BK / 16; ++kb) {
            f32x4 a[TM], b[TN];
            for (int i = 0; i < TM; ++i) a[i] = *(const f32x4 *) &st[at((wm * TM + i) * 16 + lr, 4 * kb + lg)];
            for (int j = 0; j < TN; ++j) b[j] = *(const f32x4 *) &st[at(BM + (wn * TN + j) * 16 + lr, 4 * kb + lg)];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                for (int i = 0; i < TM; ++i)
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][t], b[j][t], acc[i][j], 0, 0, 0);
        }
    }
    __syncthreads();   // the ring's last reads are done: the epilogue reuses the LDS
    f32_epilogue<TM, TN, YBF16, SNAKE>(p, sk, acc, smem, bm0, bn0, z);
}

template <int TM, int TN>
void launch_tiles(const GemmProblem &p, int y_bf16, hipStream_t s, const F32Snake *snake) {
    constexpr int BM = 2 * TM * 16, BN = 2 * TN * 16;
    dim3 grid((p.M + BM - 1) / BM, (p.N + BN - 1) / BN, p.splits > 1 ? p.splits : 1);
    const F32Snake none = {nullptr, nullptr, nullptr, 1};
    if (y_bf16) launch_kernel((gemm_f32_kernel<TM, TN, true, false>), grid, dim3(NT), 0, s, p, none);
    else if (snake) launch_kernel((gemm_f32_kernel<TM, TN, false, true>), grid, dim3(NT), 0, s, p, *snake);
    else launch_kernel((gemm_f32_kernel<TM, TN, false, false>), grid, dim3(NT), 0, s, p, none);
}

template <int TM, int TN, int NS>
void launch_tiles_dl(const GemmProblem &p, int y_bf16, hipStream_t s, const F32Snake *snake, uint32_t x_bytes) {
    constexpr int BM = 2 * TM * 16, BN = 2 * TN * 16;
    dim3 grid((p.M + BM - 1) / BM, (p.N + BN - 1) / BN, p.splits > 1 ? p.splits : 1);
    const F32Snake none = {nullptr, nullptr, nullptr, 1};
    if (y_bf16) launch_kernel((gemm_f32_dl_kernel<TM, TN, NS, true, false>), grid, dim3(NT), 0, s, p, none, x_bytes);
    else if (snake) launch_kernel((gemm_f32_dl_kernel<TM, TN, NS, false, true>), grid, dim3(NT), 0, s, p, *snake, x_bytes);
    else launch_kernel((gemm_f32_dl_kernel<TM, TN, NS, false, false>), grid, dim3(NT), 0, s, p, none, x_bytes);
}

// bytes of the activation operand the direct-load kernel may read, or 0 when
// it does not take the problem: 16-byte aligned rows and chunks (K, the
// convolution's input channels and every stride a multiple of 4 floats,
// whole 32-wide K steps inside one kernel tap), plain or implicit-im2col rows,
// 31-bit byte ranges for the buffer descriptors
uint32_t dl_x_bytes(const GemmProblem &p) {
    const uintptr_t al = (uintptr_t) p.x | (uintptr_t) p.wf;
    if (p.K % BK || p.ld_w % 4 || p.ld_x % 4 || al % 16 || p.x_group_rows) return 0;
    if ((int64_t) p.M * p.ld_w * 4 >= ((int64_t) 1 << 31)) return 0;
    int64_t xb;
    if (p.conv_ic) {
        if (p.conv_ic % BK || p.x_group_stride % 4) return 0;
        const int64_t items = p.N / p.conv_ow;
        xb = ((items - 1) * p.x_group_stride + (int64_t) (p.conv_iw - 1) * p.ld_x + p.conv_ic) * 4;
    } else {
        if (p.ld_x < p.K) return 0;
        xb = ((int64_t) (p.N - 1) * p.ld_x + p.K) * 4;
    }
    return xb < ((int64_t) 1 << 31) ? (uint32_t) xb : 0;
}

}  // namespace

hipError_t launch_gemm_f32(const GemmProblem &p, int y_bf16, hipStream_t s, const F32Snake *snake) {
    if (p.M < 1 || p.N < 1 || p.K < 4 || (p.K & 3) || !p.wf || (p.accumulate && y_bf16)) return hipErrorInvalidValue;
    // split-K slices [splits][N][ld_y] of f32 partial sums: no bias, epilogue or accumulation
    const int S = p.splits > 1 ? p.splits : 1;
    if (S > 1 && (S > (p.K + 31) / 32 || p.bias || snake || y_bf16 || p.accumulate)) return hipErrorInvalidValue;
    if (snake && (y_bf16 || !snake->ea || !snake->eb || snake->period < 4 || snake->period % 4 || p.M % snake->period))
        return hipErrorInvalidValue;
    if (p.conv_ic && (p.conv_ic % 4 || p.K % p.conv_ic || p.x_group_rows || p.conv_ow < 1 || p.conv_iw < 1 ||
                      p.conv_s < 1 || p.conv_d < 1 || p.conv_p < 0 || p.N % p.conv_ow))
        return hipErrorInvalidValue;
    // 128 x 128 workgroup tiles (4 x 4 per wave, 72 KiB of LDS: two workgroups
    // per CU) where there are enough such tiles: unsplit products (the VAE's
    // convolutions, k7 at 128-1024 channels 62.5-67.7 -> 69.7-74.2 % of the
    // fp32 peak) and wide ones in slices of >= 768 k (the graph's 30 s convMLP
    // w1 / w3, 2816 outputs, K = 3072 in 4 slices: 257 -> 235 us). 128 x 64
    // otherwise: K-split products with 1024 outputs (the graph's w2 in 8
    // slices: 255 us against 304) and few tiles. Every tile shape sums each
    // output in the same order: the same bits.
    int tile = tuning().f32_tile;
    if (tile == 0) {
        const int64_t tiles44 = (int64_t) ((p.M + 127) / 128) * ((p.N + 127) / 128) * S;
        tile = (tiles44 >= tuning().f32_t44 && (S == 1 || (p.K / S >= 768 && p.M >= 2048))) ? 44 : 42;
    }
    // direct global -> LDS loads with a two-stage ring where the operands
    // allow (the same bits; 3-10 % faster than register staging on the VAE's
    // and the graph's convolutions; a three-stage ring keeps one 128 x 128
    // workgroup per CU and is 10-15 % slower)
    const uint32_t xb = tuning().f32_dl ? dl_x_bytes(p) : 0;
    if (xb) {
        const int ns = tuning().f32_dl_ns == 3 ? 3 : 2;
        if (tile == 44) ns == 2 ? launch_tiles_dl<4, 4, 2>(p, y_bf16, s, snake, xb) : launch_tiles_dl<4, 4, 3>(p, y_bf16, s, snake, xb);
        else ns == 2 ? launch_tiles_dl<4, 2, 2>(p, y_bf16, s, snake, xb) : launch_tiles_dl<4, 2, 3>(p, y_bf16, s, snake, xb);
        return hipGetLastError();
    }
    switch (tile) {
        case 44: launch_tiles<4, 4>(p, y_bf16, s, snake); break;
        case 24: launch_tiles<2, 4>(p, y_bf16, s, snake); break;
        case 22: launch_tiles<2, 2>(p, y_bf16, s, snake); break;
        default: launch_tiles<4, 2>(p, y_bf16, s, snake); break;
    }
    return hipGetLastError();
}

}  // namespace tsk
