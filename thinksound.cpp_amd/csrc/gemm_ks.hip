// gemm_ks.hip — BF16 weight GEMMs of the MM-DiT block projections on gfx950
// (the ggml_mul_mat nodes of lin(), src/mmdit.cpp:12-25), one launch for up
// to two independent problems (the latent and text streams of a joint block):
//
//   Y[n, m] = epi( sum_k X[n, k] * W[m, k] + bias[m] )
//
// Work split. A workgroup of four waves owns a BM x BN output tile (BM
// weight rows, BN tokens) over its K range (a K slice when the caller asks
// for split-K partials). The K range is cut into 32-wide stages and wave w
// takes stages w, w + 4, w + 8, ...: the four waves compute the same tile on
// disjoint K, so no wave ever reads another wave's operands. Each wave
// streams its stages into a private LDS ring (R stages deep) with direct
// global->LDS loads and waits only on its own load counter: the main loop
// has no barrier, and R stages of every wave (up to 144 KiB per CU) are in
// flight at once, which is what hides L2 / HBM latency at these thin shapes.
//
// Operand layout. A stage holds TM A fragments (16 weight rows x 32 k each,
// 1 KiB, read as is from the MFMA-tiled weight layout of tiled_index()) and
// TN B fragments (16 tokens x 32 k: lane l fetches token l % 16, k 8 (l / 16)
// + 0..7, 16 bytes of a bf16 activation row). Both land in LDS in the lane
// order of the v_mfma_f32_16x16x32_bf16 operands, so every fragment is one
// conflict-free ds_read_b128 at lane * 16.
//
// Cooperative tiles (MODE_COOP, for token counts that fill the chip with
// 128-token tiles): the four waves split the output tile 2 x 2 instead and
// share one LDS ring of 32-wide stages, each wave loading a quarter of every
// stage's fragments; a stage is consumed after every wave's loads of it have
// landed (own load counter, then one barrier per stage). Each wave then
// reads (TM + TN) / 2 fragments for TM * TN / 4 MFMAs, half the LDS traffic
// per MFMA of the K-split tiles, and no partial tiles need summing.
//
// The four partial tiles are summed through LDS in wave order 0, 1, 2, 3:
// every output element is summed in the same order whatever the launch
// shape, the token count or its tile position, so batch rows are
// independent bit for bit. The epilogue runs on the summed tile: f32 / bf16
// store (+bias), GELU(tanh) -> bf16, split-K partial slices (summed in fixed
// order by their consumer), or the QKV epilogue (RMSNorm * w on q and k,
// RoPE from a cos/sin table on the latent stream, the fp16 cast into the
// attention layout [B][n_head][Ntot][64] and V^T, mmdit.cpp:78-90).
#include <cstdlib>

#include "tsk_common.h"
#include "tsk_internal.h"
#include "tsk_runtime.h"

namespace tsk {

namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int NT = 256;   // 4 waves

// 16 bytes per lane from global memory straight into LDS at lds_base + lane * 16
__device__ __forceinline__ void g2l16(const void *src, void *lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_void *) lds_base, 16, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// The same waits as s_waitcnt instructions the compiler sees (its own
// counter bookkeeping then knows what has completed): vmcnt(N) only, and
// lgkmcnt(0) only (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8; a field at its maximum does not wait).
template <int N>
__device__ __forceinline__ void wait_vm_seen() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_lgkm0_seen() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

template <int L, int R>
__device__ __forceinline__ void wait_stages_seen(int rem) {
    if constexpr (R >= 4) {
        if (rem >= 3) { wait_vm_seen<3 * L>(); return; }
    }
    if constexpr (R >= 3) {
        if (rem >= 2) { wait_vm_seen<2 * L>(); return; }
    }
    if (rem >= 1) { wait_vm_seen<L>(); return; }
    wait_vm_seen<0>();
}

// wait until at most `rem` stages of L loads each are still in flight
template <int L, int R>
__device__ __forceinline__ void wait_stages(int rem) {
    if constexpr (R >= 4) {
        if (rem >= 3) { wait_vm<3 * L>(); return; }
    }
    if constexpr (R >= 3) {
        if (rem >= 2) { wait_vm<2 * L>(); return; }
    }
    if (rem >= 1) { wait_vm<L>(); return; }
    wait_vm<0>();
}

struct Coord {
    int pi, tm, tn, split;
};

// Workgroup -> (problem, m tile, n tile, split). Problems start at multiples of
// 8 so that bid % 8 (the XCD the workgroup lands on) is the same in both
// numberings. When the (m tile, split) pairs divide evenly over the 8 XCDs,
// XCD x owns the pairs c = x, x + 8, ... with c = m tile * splits + split and
// runs every token tile of each: a weight tile is fetched into one XCD's L2
// only, and with splits dividing 8 an XCD reads a single K slice of the
// activations instead of all of them. `li` counts the problem's workgroups.
__device__ __forceinline__ bool decode(const GemmProblem &p, int li, Coord &c) {
    const int cols = p.tiles_n * p.splits;
    if (li >= p.tiles_m * cols) return false;
    if (((p.tiles_m * p.splits) & 7) == 0) {
        const int s = li >> 3;
        const int pair = (li & 7) + 8 * (s / p.tiles_n);
        c.tn = s % p.tiles_n;
        c.tm = pair / p.splits;
        c.split = pair % p.splits;
    } else {
        c.tm = li % p.tiles_m;
        const int col = li / p.tiles_m;
        c.tn = col % p.tiles_n;
        c.split = col / p.tiles_n;
    }
    return true;
}

__device__ __forceinline__ int64_t x_row(const GemmProblem &p, int n) {
    return p.x_group_rows ? (int64_t) (n / p.x_group_rows) * p.x_group_stride + (int64_t) (n % p.x_group_rows) * p.ld_x
                          : (int64_t) n * p.ld_x;
}

// main-loop modes
enum : int {
    MODE_RING = 0,     // K-split waves, private LDS rings of direct global->LDS loads
    MODE_DIRECT = 1,   // K-split waves, operands straight into registers
    MODE_COOP = 2,     // 2 x 2 waves over the tile, one shared LDS ring
    MODE_COOP_PIPE = 3,// MODE_COOP with the next stage's fragments read from LDS during this stage's MFMAs
    MODE_COOP64 = 4,   // MODE_COOP with 64-wide k stages of whole 128-byte rows (swizzled in LDS)
    MODE_PF = 5        // MODE_COOP64's LDS layout, double-buffered, fed from R stages of register prefetch
};

template <int TM, int TN, int R, int MODE, int KH = 1>
constexpr size_t lds_bytes() {
    constexpr bool coop = MODE == MODE_COOP || MODE == MODE_COOP_PIPE || MODE == MODE_COOP64 || MODE == MODE_PF;
    constexpr size_t ring = MODE == MODE_DIRECT ? 0
                          : MODE == MODE_PF     ? (size_t) 2 * 2 * (TM + TN) * 1024
                          : MODE == MODE_COOP64 ? (size_t) R * 2 * (TM + TN) * 1024
                          : coop                ? (size_t) R * KH * (TM + TN) * 1024
                                                : (size_t) 4 * R * (TM + TN) * 1024;
    constexpr size_t red = coop ? (size_t) (16 * TN) * (16 * TM + 4) * 4
                                : (size_t) 4 * (16 * (TN < 4 ? TN : 4)) * (16 * TM + 4) * 4;
    return ring > red ? ring : red;
}

// read by fragments of the implicit im2col that fall into the zero padding
__device__ __attribute__((aligned(16))) uint16_t g_zero_row[64];

constexpr bool epi_swiglu(int epi) { return epi == EPI_SWIGLU_F32 || epi == EPI_SWIGLU_BF16; }

// The tile of one problem; `p` is the kernel argument itself (g.p[0] or
// g.p[1] by name, never by a runtime index), so every field is read at a fixed
// kernel-argument offset and all of them can be requested at kernel entry.
template <int TM, int TN, int R, int MODE, int EPI, int KH, bool CONV>
__device__ __forceinline__ void gemm_ks_tile(const GemmProblem &p, const Coord tc, uint8_t *lds) {
    constexpr int BM = 16 * TM, BN = 16 * TN, L = TM + TN, STAGE = KH * L * 1024;
    constexpr bool PIPE = MODE == MODE_COOP_PIPE, PF = MODE == MODE_PF, C64 = MODE == MODE_COOP64 || PF;
    constexpr bool COOP = MODE == MODE_COOP || PIPE || C64, DIRECT = MODE == MODE_DIRECT;
    static_assert(!COOP || (TM % 2 == 0 && TN % 2 == 0 && (C64 ? L % 2 : L % 4) == 0), "cooperative tile shape");
    static_assert((COOP && !PIPE && !C64) || KH == 1, "KH: 32-wide k tiles per cooperative stage");
    static_assert(!PIPE || R >= 3, "pipelined fragments need three ring slots");
    static_assert(COOP || (!CONV && !epi_swiglu(EPI)), "convolutions and SwiGLU run cooperative tiles");
    constexpr int TMW = COOP ? TM / 2 : TM, TNW = COOP ? TN / 2 : TN;   // 16x16 tiles per wave
    // SwiGLU: row blocks [0, TM / 2) of the tile are W's, [TM / 2, TM) the
    // same rows of W3, so the tile holds BM / 2 output features
    constexpr bool SWIGLU = epi_swiglu(EPI);
    constexpr int BMO = SWIGLU ? BM / 2 : BM;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int bm0 = tc.tm * BMO, bn0 = tc.tn * BN;
    const int KT = p.K >> 5;                                  // 32-wide k tiles
    const int kt0 = tc.split * p.kt_split, kt1 = min(KT, kt0 + p.kt_split);
    const int nst = kt1 - kt0;
    const int my_n = C64 ? nst / 2 : COOP ? nst / KH : nst > wave ? (nst - wave + 3) >> 2 : 0;   // stages this wave computes
    const int wm = COOP ? (wave & 1) : 0, wn = COOP ? (wave >> 1) : 0;       // cooperative quadrant

    // A: tile (rb, kt) of the tiled weights at (rb * KT + kt) * 512 elements,
    // this lane's 16 bytes at lane * 8; row-major weights (cooperative tiles
    // only): row 16 rb + l % 16, k 32 kt + 8 (l / 16). Row blocks past M read
    // the last one (their outputs are never stored).
    const uint16_t *abase[TM];
    const int astep = p.w_tiled ? 512 : 32;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int rb = min((bm0 >> 4) + (SWIGLU ? i % (TM / 2) : i), (p.M >> 4) - 1);
        const uint16_t *wsrc = SWIGLU && i >= TM / 2 ? p.w3 : p.w;
        abase[i] = p.w_tiled ? wsrc + (int64_t) rb * KT * 512 + lane * 8
                             : wsrc + (int64_t) (rb * 16 + (lane & 15)) * p.ld_w + 8 * (lane >> 4);
    }
    // B: token bn0 + 16 j + l % 16 (tokens past N read row N - 1), k 8 (l / 16);
    // implicit im2col: the token is output position ow of batch item b, and
    // k tile kt reads input position ow s + kw d - p (kw = 32 kt / IC), or a
    // zero row in the padding
    const uint16_t *bsrc[TN];
    int biw[CONV ? TN : 1];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int n = min(bn0 + 16 * j + (lane & 15), p.N - 1);
        if constexpr (CONV) {
            const int b = n / p.conv_ow, ow = n - b * p.conv_ow;
            bsrc[j] = (const uint16_t *) p.x + (int64_t) b * p.x_group_stride + 8 * (lane >> 4);
            biw[j] = ow * p.conv_s - p.conv_p;
        } else {
            bsrc[j] = (const uint16_t *) p.x + x_row(p, n) + 8 * (lane >> 4);
        }
    }
    auto bfrag = [&](int j, int kt) -> const uint16_t * {
        if constexpr (CONV) {
            const int k = kt * 32, kw = k / p.conv_ic, ic0 = k - kw * p.conv_ic;
            const int iw = biw[j] + kw * p.conv_d;
            return iw >= 0 && iw < p.conv_iw ? bsrc[j] + (int64_t) iw * p.ld_x + ic0 : g_zero_row + 8 * (lane >> 4);
        } else {
            return bsrc[j] + kt * 32;
        }
    };
    uint8_t *ring = lds + wave * (R * STAGE);
    auto issue = [&](int t, int slot) {
        const int kt = kt0 + wave + 4 * t;
        uint8_t *dst = ring + slot * STAGE;
#pragma unroll
        for (int i = 0; i < TM; ++i)
            g2l16(abase[i] + (int64_t) kt * astep, dst + i * 1024);
#pragma unroll
        for (int j = 0; j < TN; ++j)
            g2l16(bfrag(j, kt), dst + (TM + j) * 1024);
    };

    f32x4 acc[TMW][TNW];
#pragma unroll
    for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    if constexpr (C64) {
        // Stages of 64 k (k tiles kt0 + 2 t, + 1; the launcher checks that
        // every K range holds an even number of tiles). A stage holds TM + TN
        // units of 2 KiB: tiled weights as two 1 KiB MFMA fragments (k tile
        // 2 t, 2 t + 1); row-major weights and activations as 16 rows x 128
        // bytes, loaded as two blocks of 8 rows in which lane i fetches row
        // 8 h + i / 8, 16-byte chunk (i % 8) ^ key, key = (i / 8) ^ 4 h: each
        // row is one whole 128-byte line, and the MFMA read of chunk c of
        // row t at block t / 8, row t % 8, slot c ^ key hits 16 distinct
        // 16-byte bank groups over the 16 rows.
        constexpr int U = TM + TN, LW = 2 * U / 4;
        constexpr int USZ = 2048, STG = U * USZ;
        const int ns = my_n;
        const int r8 = lane >> 3;
        // MFMA read offsets of this lane (token / row t = lane % 16, chunk 4 kh + lane / 16)
        int roff[2];
        {
            const int tq = lane & 15, kc = lane >> 4;
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
                roff[kh] = (tq >> 3) * 1024 + (tq & 7) * 128 + (((4 * kh + kc) ^ (tq & 7) ^ (4 * (tq >> 3))) * 16);
        }
        // this wave's loads, fixed per q for the whole K range: fragment
        // f = wave + 4 q is unit f / 2, half f % 2; its source advances by
        // `step` elements per stage (1024 for tiled weights, 64 otherwise).
        // Row-major operands: lane i of half h fetches row 8 h + i / 8 of its
        // 16-row block, bf16 chunk qchk = (i % 8) ^ (i / 8) ^ 4 h. Every source
        // is computed from (u, h) directly: the unit and half depend on the
        // wave, and arrays indexed by them would live in scratch memory.
        const uint16_t *qsrc[LW];
        int qlds[LW], qstep[LW], qconv[CONV ? LW : 1], qchk[CONV ? LW : 1];
#pragma unroll
        for (int q = 0; q < LW; ++q) {
            const int f = wave + 4 * q, u = f >> 1, h = f & 1;
            const int chk = ((lane & 7) ^ r8 ^ (4 * h)) * 8;            // bf16 elements
            qlds[q] = u * USZ + h * 1024;
            if constexpr (CONV) {
                qconv[q] = 0;
                qchk[q] = chk;
            }
            if (u < TM) {
                const int rb = min((bm0 >> 4) + (SWIGLU ? u % (TM / 2) : u), (p.M >> 4) - 1);
                const uint16_t *wsrc = SWIGLU && u >= TM / 2 ? p.w3 : p.w;
                if (p.w_tiled) {
                    qsrc[q] = wsrc + (int64_t) rb * KT * 512 + lane * 8 + (int64_t) (kt0 + h) * 512;
                    qstep[q] = 1024;
                } else {
                    qsrc[q] = wsrc + (int64_t) (rb * 16 + 8 * h + r8) * p.ld_w + chk + kt0 * 32;
                    qstep[q] = 64;
                }
            } else {
                const int n = min(bn0 + 16 * (u - TM) + 8 * h + r8, p.N - 1);
                if constexpr (CONV) {
                    // implicit im2col: the row base (batch item) and first input position
                    const int b = n / p.conv_ow, ow = n - b * p.conv_ow;
                    qsrc[q] = (const uint16_t *) p.x + (int64_t) b * p.x_group_stride + chk;
                    qconv[q] = ow * p.conv_s - p.conv_p;
                    qstep[q] = 0;
                } else {
                    qsrc[q] = (const uint16_t *) p.x + x_row(p, n) + chk + kt0 * 32;
                    qstep[q] = 64;
                }
            }
        }
        const bool qisb[4] = {(wave + 0) / 2 >= TM, (wave + 4) / 2 >= TM, (wave + 8) / 2 >= TM, (wave + 12) / 2 >= TM};
        auto cissue = [&](int t, int slot) {
            uint8_t *dst = lds + slot * STG;
#pragma unroll
            for (int q = 0; q < LW; ++q) {
                if constexpr (CONV) {
                    const bool isb = q < 4 ? qisb[q] : (wave + 4 * q) / 2 >= TM;
                    if (isb) {
                        const int k = (kt0 + 2 * t) * 32, kw = k / p.conv_ic, ic0 = k - kw * p.conv_ic;
                        const int iw = qconv[q] + kw * p.conv_d;
                        g2l16(iw >= 0 && iw < p.conv_iw ? qsrc[q] + (int64_t) iw * p.ld_x + ic0 : g_zero_row + qchk[q],
                              dst + qlds[q]);
                        continue;
                    }
                }
                g2l16(qsrc[q] + (int64_t) t * qstep[q], dst + qlds[q]);
            }
        };
        // A fragment read offsets: tiled (lane order) or swizzled rows
        int aro[2];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) aro[kh] = p.w_tiled ? kh * 1024 + lane * 16 : roff[kh];
        // every fragment of the stage is read before the first MFMA (the
        // scheduling barrier keeps the compiler from interleaving reads and
        // MFMAs, which serialises on the LDS latency): the second half's reads
        // are in flight during the first half's MFMAs
        auto compute = [&](const uint8_t *src) {
            bf16x8 a[2][TMW], b[2][TNW];
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
                for (int i = 0; i < TMW; ++i) a[kh][i] = *(const bf16x8 *) (src + (wm * TMW + i) * USZ + aro[kh]);
#pragma unroll
                for (int j = 0; j < TNW; ++j) b[kh][j] = *(const bf16x8 *) (src + (TM + wn * TNW + j) * USZ + roff[kh]);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kh = 0; kh < 2; ++kh)
#pragma unroll
                for (int i = 0; i < TMW; ++i)
#pragma unroll
                    for (int j = 0; j < TNW; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[kh][i], b[kh][j], acc[i][j], 0, 0, 0);
        };
        if constexpr (PF) {
            // R stages of this wave's loads in flight in registers; LDS holds
            // two stages (the one being read, the one being written). Every
            // iteration issues one stage's loads unconditionally (past the
            // last stage it re-reads the last one), so the count of loads in
            // flight is the same on every trip and the compiler's own counter
            // waits (before each LDS write of a register set) wait for exactly
            // one stage.
            u32x4 rg[R][LW];
            auto gload = [&](int t, int set) {
                t = min(t, ns - 1);
#pragma unroll
                for (int q = 0; q < LW; ++q) {
                    const uint16_t *src = qsrc[q] + (int64_t) t * qstep[q];
                    if constexpr (CONV) {
                        const bool isb = q < 4 ? qisb[q] : (wave + 4 * q) / 2 >= TM;
                        if (isb) {
                            const int k = (kt0 + 2 * t) * 32, kw = k / p.conv_ic, ic0 = k - kw * p.conv_ic;
                            const int iw = qconv[q] + kw * p.conv_d;
                            src = iw >= 0 && iw < p.conv_iw ? qsrc[q] + (int64_t) iw * p.ld_x + ic0 : g_zero_row + qchk[q];
                        }
                    }
                    rg[set][q] = *(const u32x4 *) src;
                }
            };
            auto swrite = [&](int set, int slot) {
                uint8_t *dst = lds + slot * STG + lane * 16;
#pragma unroll
                for (int q = 0; q < LW; ++q) *(u32x4 *) (dst + qlds[q]) = rg[set][q];
            };
            if (ns > 0) {
#pragma unroll
                for (int s = 0; s < R; ++s) gload(s, s);
                swrite(0, 0);
                gload(R, 0);
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                // trip t reads stage t from slot t % 2, writes stage t + 1 from
                // register set (t + 1) % R into the other slot, refills that
                // set with stage t + 1 + R; the barrier ends every wave's reads
                // of slot t % 2 before trip t + 1 overwrites it. Trips run R at
                // a time so that every register set index is a constant (a
                // register array indexed at run time would live in scratch).
                // The LDS writes and refills are unconditional (past the last
                // stage they move copies of it that nobody reads): the same
                // loads are in flight on every path, so the compiler's counter
                // wait before each write lets R - 1 stages stay in flight.
                for (int t0 = 0; t0 < ns; t0 += R) {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const int t = t0 + r;
                        if (t < ns) compute(lds + (t & 1) * STG);
                        swrite((r + 1) % R, (t + 1) & 1);
                        gload(t + 1 + R, (r + 1) % R);
                        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                    }
                }
            }
        } else {
#pragma unroll
        for (int s = 0; s < R - 1; ++s)
            if (s < ns) cissue(s, s);
        int slot = 0;
        for (int t = 0; t < ns; ++t) {
            wait_stages<LW, R - 1>(min(ns - 1 - t, R - 2));
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (t + R - 1 < ns) cissue(t + R - 1, slot == 0 ? R - 1 : slot - 1);
            compute(lds + slot * STG);
            slot = slot + 1 == R ? 0 : slot + 1;
        }
        }
    } else if constexpr (PIPE) {
        // shared ring as below (KH = 1); the fragments of stage t + 1 are read
        // into a second register set while stage t's MFMAs run, so the LDS
        // latency overlaps the MFMAs. Slot of stage t - 1 (read during
        // iteration t - 2) is refilled at iteration t.
        constexpr int LW = L / 4;
        const int ns = my_n;
        auto cissue = [&](int t, int slot) {
            uint8_t *dst = lds + slot * STAGE;
            const int kt = kt0 + t;
#pragma unroll
            for (int q = 0; q < LW; ++q) {
                const int f = wave + 4 * q;
                if (f < TM) g2l16(abase[f] + (int64_t) kt * astep, dst + f * 1024);
                else g2l16(bfrag(f - TM, kt), dst + f * 1024);
            }
        };
        bf16x8 a0[TMW], b0[TNW], a1[TMW], b1[TNW];
        auto cread = [&](int slot, bf16x8 (&a)[TMW], bf16x8 (&b)[TNW]) {
            const uint8_t *src = lds + slot * STAGE + lane * 16;
#pragma unroll
            for (int i = 0; i < TMW; ++i) a[i] = *(const bf16x8 *) (src + (wm * TMW + i) * 1024);
#pragma unroll
            for (int j = 0; j < TNW; ++j) b[j] = *(const bf16x8 *) (src + (TM + wn * TNW + j) * 1024);
        };
#pragma unroll
        for (int s = 0; s < R - 1; ++s)
            if (s < ns) cissue(s, s);
        if (ns > 0) {
            wait_stages_seen<LW, R - 1>(min(ns - 1, R - 2));
            wait_lgkm0_seen();
            asm volatile("s_barrier" ::: "memory");
            cread(0, a0, b0);
        }
        int slot = 0;
        // the two register sets alternate (two iterations per loop trip), so
        // the fragments being read are never the MFMAs' operands and the
        // compiler's counter waits let the reads stay in flight
        auto step = [&](int t, const bf16x8 (&ac)[TMW], const bf16x8 (&bc)[TNW], bf16x8 (&an)[TMW],
                        bf16x8 (&bn)[TNW]) {
            const int nslot = slot + 1 == R ? 0 : slot + 1;
            if (t + 1 < ns) {
                // stage t + 1 has landed for every wave, and every wave is
                // done with iteration t - 1 (its reads of stage t)
                wait_stages_seen<LW, R - 1>(min(ns - 2 - t, R - 3));
                wait_lgkm0_seen();
                asm volatile("s_barrier" ::: "memory");
                cread(nslot, an, bn);
                if (t + R - 1 < ns) cissue(t + R - 1, slot == 0 ? R - 1 : slot - 1);
            }
#pragma unroll
            for (int i = 0; i < TMW; ++i)
#pragma unroll
                for (int j = 0; j < TNW; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ac[i], bc[j], acc[i][j], 0, 0, 0);
            slot = nslot;
        };
        // in the loop both steps read ahead (provably, so the compiler's
        // waits stay exact); the last one or two steps follow it
        int t = 0;
        for (; t + 2 < ns; t += 2) {
            step(t, a0, b0, a1, b1);
            step(t + 1, a1, b1, a0, b0);
        }
        if (t < ns) step(t, a0, b0, a1, b1);
        if (t + 1 < ns) step(t + 1, a1, b1, a0, b0);
    } else if constexpr (COOP) {
        // shared ring of R stages of KH 32-wide k tiles (the launcher checks
        // that KH divides the tiles of every K range); wave w loads fragments
        // w, w + 4, ... of each stage, fragment h * L + f being tile h's A
        // fragment f (f < TM) or B fragment f - TM
        constexpr int LW = KH * L / 4;
        const int ns = my_n;
        auto cissue = [&](int t, int slot) {
            uint8_t *dst = lds + slot * STAGE;
#pragma unroll
            for (int q = 0; q < LW; ++q) {
                const int fq = wave + 4 * q, h = fq / L, f = fq % L;
                const int kt = kt0 + t * KH + h;
                if (f < TM) g2l16(abase[f] + (int64_t) kt * astep, dst + fq * 1024);
                else g2l16(bfrag(f - TM, kt), dst + fq * 1024);
            }
        };
#pragma unroll
        for (int s = 0; s < R - 1; ++s)
            if (s < ns) cissue(s, s);
        int slot = 0;
        for (int t = 0; t < ns; ++t) {
            // this wave's loads of stage t have landed; the barrier makes every
            // wave's visible and ends every wave's reads of stage t - 1, whose
            // slot is refilled next
            wait_stages<LW, R - 1>(min(ns - 1 - t, R - 2));
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (t + R - 1 < ns) cissue(t + R - 1, slot == 0 ? R - 1 : slot - 1);
#pragma unroll
            for (int h = 0; h < KH; ++h) {
                const uint8_t *src = lds + slot * STAGE + h * (L * 1024) + lane * 16;
                bf16x8 a[TMW], b[TNW];
#pragma unroll
                for (int i = 0; i < TMW; ++i) a[i] = *(const bf16x8 *) (src + (wm * TMW + i) * 1024);
#pragma unroll
                for (int j = 0; j < TNW; ++j) b[j] = *(const bf16x8 *) (src + (TM + wn * TNW + j) * 1024);
#pragma unroll
                for (int i = 0; i < TMW; ++i)
#pragma unroll
                    for (int j = 0; j < TNW; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
            slot = slot + 1 == R ? 0 : slot + 1;
        }
    } else if constexpr (DIRECT) {
        // operands straight into registers, R stages in flight. The stage
        // count of every wave is a multiple of R (checked by the launcher), so
        // every refill below is a real stage and the loads are unconditional:
        // the compiler's load counter then waits for exactly one stage.
        u32x4 ra[R][TM], rb[R][TN];
        auto dload = [&](int t, int set) {
            const int kt = kt0 + wave + 4 * t;
#pragma unroll
            for (int i = 0; i < TM; ++i) ra[set][i] = *(const u32x4 *) (abase[i] + (int64_t) kt * astep);
#pragma unroll
            for (int j = 0; j < TN; ++j) rb[set][j] = *(const u32x4 *) bfrag(j, kt);
        };
        auto consume = [&](int set) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, ra[set][i]), __builtin_bit_cast(bf16x8, rb[set][j]), acc[i][j], 0, 0, 0);
        };
        if (my_n > 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) dload(r, r);
            for (int t0 = 0; t0 < my_n - R; t0 += R) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    consume(r);
                    dload(t0 + r + R, r);
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r) consume(r);
        }
    } else {
#pragma unroll
    for (int s = 0; s < R; ++s)
        if (s < my_n) issue(s, s);
    int slot = 0;
    for (int t = 0; t < my_n; ++t) {
        wait_stages<L, R>(min(my_n - 1 - t, R - 1));
        const uint8_t *src = ring + slot * STAGE + lane * 16;
        bf16x8 a[TM], b[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = *(const bf16x8 *) (src + i * 1024);
#pragma unroll
        for (int j = 0; j < TN; ++j) b[j] = *(const bf16x8 *) (src + (TM + j) * 1024);
        // the slot is refilled next: its reads must have returned
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (t + R < my_n) issue(t + R, slot);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        slot = slot + 1 == R ? 0 : slot + 1;
    }
    }

    // ---- sum the four waves' partial tiles, 64 tokens at a time: red[w][token][feature]
    // (cooperative tiles: each wave stores its quadrant of one [token][feature] tile)
    constexpr int LDY = BM + 4;
    constexpr int TNC = COOP ? TN : TN < 4 ? TN : 4, BNC = 16 * TNC;
    float *red = (float *) lds;
#pragma unroll
    for (int c = 0; c < TN / TNC; ++c) {
    const int bn0c = bn0 + c * BNC;
    __syncthreads();                                          // rings drained / previous chunk consumed
    if constexpr (COOP) {
#pragma unroll
        for (int i = 0; i < TMW; ++i)
#pragma unroll
            for (int j = 0; j < TNW; ++j)
                *(f32x4 *) &red[(16 * (wn * TNW + j) + (lane & 15)) * LDY + 16 * (wm * TMW + i) + 4 * (lane >> 4)] =
                    acc[i][j];
    } else {
        float *mine = red + wave * (BNC * LDY);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TNC; ++j)
                *(f32x4 *) &mine[(16 * j + (lane & 15)) * LDY + 16 * i + 4 * (lane >> 4)] = acc[i][c * TNC + j];
    }
    __syncthreads();
    auto sum4 = [&](int nl, int ml) -> f32x4 {
        const float *r0 = red + nl * LDY + ml;
        f32x4 v = *(const f32x4 *) r0;
        if constexpr (!COOP) {
#pragma unroll
            for (int w = 1; w < 4; ++w) {
                const f32x4 u = *(const f32x4 *) (r0 + w * (BNC * LDY));
                v = f32x4{v[0] + u[0], v[1] + u[1], v[2] + u[2], v[3] + u[3]};
            }
        }
        return v;
    };

    auto sum1 = [&](int nl, int ml) -> float {
        const float *r0 = red + nl * LDY + ml;
        float v = *r0;
        if constexpr (!COOP) {
#pragma unroll
            for (int w = 1; w < 4; ++w) v += r0[w * (BNC * LDY)];
        }
        return v;
    };

    if constexpr (EPI == EPI_QKV) {
        // one 16-lane group per (token, head): lane sl holds dims 4 sl .. 4 sl + 3.
        // Every global load of the epilogue (bias, norm weights, RoPE table) is
        // issued before its first store: loads and stores share one counter, so
        // a load behind a store would also wait for that store.
        const int H = p.M / 3, nh = H / 64;
        const int grp = tid >> 4, sl = tid & 15;
        constexpr int HPT = BM / 64;                 // heads per tile
        constexpr int U = BNC * HPT / (NT / 16);     // (token, head) pairs per lane group
        if (bm0 >= 2 * H && p.seq >= BNC && !p.v_rows) {
            // V tile -> V^T rows: lane (row ml, 4-position chunk) writes 4 consecutive
            // key slots of one V^T row (vt_pos keeps aligned 4-runs together), so a
            // row's 128 bytes leave as whole runs instead of 2-byte scatters. The
            // tile's tokens span at most two batch items (seq >= BNC); part 0 is
            // batch item b0 from s0, part 1 the next item from position 0.
            const int n0 = bn0c, n1 = min(bn0c + BNC, p.N);
            if (n0 < n1) {
                const int b0 = n0 / p.seq, s0 = n0 - b0 * p.seq;
                const int e0 = min(p.seq, s0 + (n1 - n0));
                const int ca0 = (p.tok_off + s0) >> 2, cnt0 = ((p.tok_off + e0 - 1) >> 2) - ca0 + 1;
                const int r1 = n1 - (b0 + 1) * p.seq;                   // tokens of item b0 + 1
                const int ca1 = p.tok_off >> 2, cnt1 = r1 > 0 ? ((p.tok_off + r1 - 1) >> 2) - ca1 + 1 : 0;
                constexpr int KR = BM / 64, CS = (BNC / 4 + 3 + 3) / 4;  // rows, chunk slots per lane
                float bv[KR];
#pragma unroll
                for (int k = 0; k < KR; ++k) bv[k] = p.bias ? p.bias[bm0 + 16 * (wave + 4 * k) + (lane & 15)] : 0.0f;
#pragma unroll
                for (int k = 0; k < KR; ++k) {
                    const int ml = 16 * (wave + 4 * k) + (lane & 15);
                    const int f = bm0 + ml - 2 * H, head = f / 64, d = f % 64;
#pragma unroll
                    for (int i = 0; i < CS; ++i) {
                        const int cj = (lane >> 4) + 4 * i;
                        if (cj >= cnt0 + cnt1) continue;
                        const int b = cj < cnt0 ? b0 : b0 + 1;
                        const int gc = cj < cnt0 ? ca0 + cj : ca1 + cj - cnt0;
                        float v[4];
                        bool all = true;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int spos = 4 * gc + e - p.tok_off, n = b * p.seq + spos;
                            const bool ok = spos >= 0 && spos < p.seq && n >= n0 && n < n1;
                            v[e] = ok ? sum1(n - n0, ml) + bv[k] : 0.0f;
                            all = all && ok;
                        }
                        uint16_t *row = p.vt + (((int64_t) b * nh + head) * 64 + d) * p.ldv + vt_pos(4 * gc);
                        if (all) {
                            const uint16_t o4[4] = {f32_to_f16_bits(v[0]), f32_to_f16_bits(v[1]),
                                                    f32_to_f16_bits(v[2]), f32_to_f16_bits(v[3])};
                            u32x2 w2;
                            __builtin_memcpy(&w2, o4, 8);
                            *(u32x2 *) row = w2;
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int spos = 4 * gc + e - p.tok_off, n = b * p.seq + spos;
                                if (spos >= 0 && spos < p.seq && n >= n0 && n < n1) row[e] = f32_to_f16_bits(v[e]);
                            }
                        }
                    }
                }
            }
        } else {
        static_assert(U * (NT / 16) == BNC * HPT, "QKV epilogue pairs");
        static_assert((NT / 16) % HPT == 0, "a lane group keeps one head");
        // lane group grp runs pairs pp = grp + 16 u: token pp / HPT, head pp % HPT
        // = grp % HPT for every u, so the bias and norm weights are one load
        const int hl = grp % HPT, f0 = bm0 + hl * 64;
        const int sec = f0 / H, head = (f0 % H) / 64;
        const f32x4 bv = p.bias ? *(const f32x4 *) (p.bias + f0 + 4 * sl) : f32x4{0, 0, 0, 0};
        const f32x4 wv = sec < 2 ? *(const f32x4 *) ((sec ? p.kn_w : p.qn_w) + 4 * sl) : f32x4{0, 0, 0, 0};
        f32x4 xs[U], css[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int nl = (grp + u * (NT / 16)) / HPT;
            const int n = bn0c + nl, spos = (n < p.N ? n : 0) % p.seq;
            xs[u] = sum4(nl, hl * 64 + 4 * sl);
            css[u] = sec < 2 && p.rope ? *(const f32x4 *) (p.rope_cs + (int64_t) spos * 64 + 4 * sl)
                                       : f32x4{0, 0, 0, 0};
        }
        // every load of the epilogue has landed before the first store (a wait
        // the compiler sees, so no per-pair wait then also waits for the
        // previous pairs' stores, which share the counter)
        __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int nl = (grp + u * (NT / 16)) / HPT;
            const int n = bn0c + nl;
            const bool live = n < p.N;
            f32x4 x = f32x4{xs[u][0] + bv[0], xs[u][1] + bv[1], xs[u][2] + bv[2], xs[u][3] + bv[3]};
            const int nn = live ? n : 0;
            const int b = nn / p.seq, spos = nn % p.seq;
            if (sec < 2) {
                // the 16 lanes of this (token, head) pair form one DPP row
                const float ss = row16_sum(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);
                const float sc = __builtin_amdgcn_rsqf(ss / 64.0f + p.eps);   // v_rsq_f32, within 1 ulp
                for (int e = 0; e < 4; ++e) x[e] = x[e] * sc * wv[e];
                if (p.rope) {
                    // (cos, sin) of pairs 2 sl, 2 sl + 1 at position spos
                    const f32x4 cs = css[u];
                    for (int q2 = 0; q2 < 2; ++q2) {
                        const float c = cs[2 * q2], sn = cs[2 * q2 + 1];
                        const float x0 = x[2 * q2], x1 = x[2 * q2 + 1];
                        x[2 * q2] = x0 * c - x1 * sn;
                        x[2 * q2 + 1] = x0 * sn + x1 * c;
                    }
                }
            }
            if (live) {
                if (sec == 0)
                    for (int e = 0; e < 4; ++e) x[e] *= p.q_scale;     // the attention's softmax scale
                uint16_t o4[4] = {f32_to_f16_bits(x[0]), f32_to_f16_bits(x[1]), f32_to_f16_bits(x[2]),
                                  f32_to_f16_bits(x[3])};
                if (sec < 2 || p.v_rows) {
                    // q, k (and V with v_rows) rows of [B][nh][Ntot][64]
                    u32x2 w2;
                    __builtin_memcpy(&w2, o4, 8);
                    uint16_t *dst = sec == 0 ? p.q : sec == 1 ? p.k : p.vt;
                    *(u32x2 *) (dst + (((int64_t) b * nh + head) * p.Ntot + p.tok_off + spos) * 64 + 4 * sl) = w2;
                } else {
                    uint16_t *vcol = p.vt + (((int64_t) b * nh + head) * 64 + 4 * sl) * p.ldv + vt_pos(p.tok_off + spos);
                    for (int e = 0; e < 4; ++e) vcol[(int64_t) e * p.ldv] = o4[e];
                }
            }
        }
        }
    } else if constexpr (SWIGLU) {
        // 8 consecutive features of one token per thread: silu(W x) * (W3 x)
        constexpr int G = BMO / 8;
        for (int it = tid; it < BNC * G; it += NT) {
            const int nl = it / G, ml = (it % G) * 8;
            const int n = bn0c + nl, m = bm0 + ml;
            if (n >= p.N || m >= p.M) continue;
            const f32x4 a0 = sum4(nl, ml), a1 = sum4(nl, ml + 4);
            const f32x4 c0 = sum4(nl, BMO + ml), c1 = sum4(nl, BMO + ml + 4);
            const float h1[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            const float h3[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
            float o[8];
            // silu(h1) = h1 / (1 + exp(-h1)), the quotient through the hardware
            // reciprocal (within 1 ulp): exp(-h1) = inf gives 0, = 0 gives h1
            for (int e = 0; e < 8; ++e) o[e] = h1[e] * __builtin_amdgcn_rcpf(1.0f + __expf(-h1[e])) * h3[e];
            if constexpr (EPI == EPI_SWIGLU_BF16) {
                uint16_t t8[8];
                for (int e = 0; e < 8; ++e) t8[e] = f32_to_bf16_bits(o[e]);
                u32x4 w;
                __builtin_memcpy(&w, t8, 16);
                *(u32x4 *) ((uint16_t *) p.y + (int64_t) n * p.ld_y + m) = w;
            } else {
                float *yr = (float *) p.y + (int64_t) n * p.ld_y + m;
                *(f32x4 *) yr = f32x4{o[0], o[1], o[2], o[3]};
                *(f32x4 *) (yr + 4) = f32x4{o[4], o[5], o[6], o[7]};
            }
        }
    } else {
        // 8 consecutive features of one token per thread; the features are
        // the same on every iteration (NT is a multiple of G), so the bias is
        // one load ahead of the loop and no store waits behind a load
        constexpr int G = BM / 8;
        static_assert(NT % G == 0, "one feature group per thread");
        f32x4 b0 = f32x4{0, 0, 0, 0}, b1 = f32x4{0, 0, 0, 0};
        if (EPI != EPI_PARTIAL && p.bias && bm0 + (tid % G) * 8 < p.M) {
            b0 = *(const f32x4 *) (p.bias + bm0 + (tid % G) * 8);
            b1 = *(const f32x4 *) (p.bias + bm0 + (tid % G) * 8 + 4);
        }
        for (int it = tid; it < BNC * G; it += NT) {
            const int nl = it / G, ml = (it % G) * 8;
            const int n = bn0c + nl, m = bm0 + ml;
            if (n >= p.N || m >= p.M) continue;
            const f32x4 v0 = sum4(nl, ml), v1 = sum4(nl, ml + 4);
            float o[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            if (EPI != EPI_PARTIAL && p.bias)
                for (int e = 0; e < 4; ++e) { o[e] += b0[e]; o[4 + e] += b1[e]; }
            if constexpr (EPI == EPI_GELU_BF16)
                for (int e = 0; e < 8; ++e) o[e] = gelu_tanh_f(o[e]);
            if constexpr (EPI == EPI_F32X) {
                // + the old y, then the SnakeBeta (the reference's order mul,
                // sin, sqr, mul, add) into y2, the split planes or y itself
                float *yr = p.y ? (float *) p.y + (int64_t) n * p.ld_y + m : nullptr;
                if (p.accumulate) {
                    const f32x4 a0 = *(const f32x4 *) yr, a1 = *(const f32x4 *) (yr + 4);
                    for (int e = 0; e < 4; ++e) { o[e] += a0[e]; o[4 + e] += a1[e]; }
                }
                if (p.snk_ea) {
                    const int P = p.snk_period, c0 = m % P;
                    const f32x4 ea0 = *(const f32x4 *) (p.snk_ea + c0), ea1 = *(const f32x4 *) (p.snk_ea + c0 + 4);
                    const f32x4 eb0 = *(const f32x4 *) (p.snk_eb + c0), eb1 = *(const f32x4 *) (p.snk_eb + c0 + 4);
                    const float ea[8] = {ea0[0], ea0[1], ea0[2], ea0[3], ea1[0], ea1[1], ea1[2], ea1[3]};
                    const float eb[8] = {eb0[0], eb0[1], eb0[2], eb0[3], eb1[0], eb1[1], eb1[2], eb1[3]};
                    float sv[8];
                    for (int e = 0; e < 8; ++e) {
                        const float sn = sinf(o[e] * ea[e]);
                        sv[e] = o[e] + (sn * sn) * eb[e];
                    }
                    if (p.yp) {
                        uint16_t hi[8], lo[8];
                        for (int e = 0; e < 8; ++e) {
                            hi[e] = f32_to_bf16_bits(sv[e]);
                            const float hf = bf16_bits_to_f32(hi[e]);
                            lo[e] = __builtin_isfinite(hf) ? f32_to_bf16_bits(sv[e] - hf) : (uint16_t) 0;
                        }
                        u32x4 wh, wl;
                        __builtin_memcpy(&wh, hi, 16);
                        __builtin_memcpy(&wl, lo, 16);
                        uint16_t *pr = p.yp + (int64_t) n * 3 * p.ld_y + (int64_t) (m / P) * 3 * P + c0;
                        *(u32x4 *) pr = wh;
                        *(u32x4 *) (pr + P) = wh;
                        *(u32x4 *) (pr + 2 * P) = wl;
                    } else if (p.y2) {
                        float *y2r = p.y2 + (int64_t) n * p.ld_y + m;
                        *(f32x4 *) y2r = f32x4{sv[0], sv[1], sv[2], sv[3]};
                        *(f32x4 *) (y2r + 4) = f32x4{sv[4], sv[5], sv[6], sv[7]};
                    } else {
                        for (int e = 0; e < 8; ++e) o[e] = sv[e];
                    }
                }
                if (yr) {
                    *(f32x4 *) yr = f32x4{o[0], o[1], o[2], o[3]};
                    *(f32x4 *) (yr + 4) = f32x4{o[4], o[5], o[6], o[7]};
                }
                continue;
            }
            if constexpr (EPI == EPI_STORE_BF16 || EPI == EPI_GELU_BF16) {
                uint16_t t8[8];
                for (int e = 0; e < 8; ++e) t8[e] = f32_to_bf16_bits(o[e]);
                u32x4 w;
                __builtin_memcpy(&w, t8, 16);
                *(u32x4 *) ((uint16_t *) p.y + (int64_t) n * p.ld_y + m) = w;
            } else {
                float *yr = (float *) p.y + (EPI == EPI_PARTIAL ? (int64_t) tc.split * p.N * p.ld_y : 0) +
                            (int64_t) n * p.ld_y + m;
                *(f32x4 *) yr = f32x4{o[0], o[1], o[2], o[3]};
                *(f32x4 *) (yr + 4) = f32x4{o[4], o[5], o[6], o[7]};
            }
        }
    }
    }   // token chunk
}

// NPROB = 1: one problem (g.p[0]); NPROB = 2: workgroups from
// g.p[1].block_begin on run the second problem
template <int TM, int TN, int R, int MODE, int EPI, int KH, bool CONV, int NPROB>
__global__ __launch_bounds__(NT) void gemm_ks_kernel(const GemmGroup g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int bid = blockIdx.x;
    Coord tc;
    if (NPROB == 2 && bid >= g.p[1].block_begin) {
        tc.pi = 1;
        if (!decode(g.p[1], bid - g.p[1].block_begin, tc)) return;
        gemm_ks_tile<TM, TN, R, MODE, EPI, KH, CONV>(g.p[1], tc, lds);
    } else {
        tc.pi = 0;
        if (!decode(g.p[0], bid, tc)) return;
        gemm_ks_tile<TM, TN, R, MODE, EPI, KH, CONV>(g.p[0], tc, lds);
    }
}

template <int TM, int TN, int R, int MODE, int EPI, int KH, bool CONV = false>
hipError_t ks_launch(GemmGroup &g, hipStream_t s) {
    constexpr int BM = 16 * TM / (epi_swiglu(EPI) ? 2 : 1), BN = 16 * TN;
    int nblocks = 0;
    for (int i = 0; i < g.nprob; ++i) {
        GemmProblem &p = g.p[i];
        p.tiles_m = (p.M + BM - 1) / BM;
        p.tiles_n = (p.N + BN - 1) / BN;
        p.kt_split = (p.K / 32 + p.splits - 1) / p.splits;
        if (KH > 1 && ((p.K / 32) % p.splits || p.kt_split % KH)) return hipErrorInvalidValue;
        if ((MODE == MODE_COOP64 || MODE == MODE_PF) &&
            ((p.K / 32) % p.splits || p.kt_split % 2 || (CONV && p.conv_ic % 64)))
            return hipErrorInvalidValue;
        p.block_begin = (nblocks + 7) & ~7;
        nblocks = p.block_begin + p.tiles_m * p.tiles_n * p.splits;
    }
    constexpr size_t lds = lds_bytes<TM, TN, R, MODE, KH>();
    static_assert(lds <= 160 * 1024, "LDS");
    auto kern = g.nprob == 2 ? gemm_ks_kernel<TM, TN, R, MODE, EPI, KH, CONV, 2>
                             : gemm_ks_kernel<TM, TN, R, MODE, EPI, KH, CONV, 1>;
    lds_opt_in((const void *) kern, lds);
    launch_kernel(kern, dim3(nblocks), dim3(NT), lds, s, g);
    return hipGetLastError();
}

template <int TM, int TN, int R, int MODE = MODE_RING, int KH = 1>
hipError_t ks_epi(GemmGroup &g, int epi, hipStream_t s) {
    switch (epi) {
        case EPI_STORE_F32: return ks_launch<TM, TN, R, MODE, EPI_STORE_F32, KH>(g, s);
        case EPI_STORE_BF16: return ks_launch<TM, TN, R, MODE, EPI_STORE_BF16, KH>(g, s);
        case EPI_GELU_BF16: return ks_launch<TM, TN, R, MODE, EPI_GELU_BF16, KH>(g, s);
        case EPI_QKV: return ks_launch<TM, TN, R, MODE, EPI_QKV, KH>(g, s);
        case EPI_PARTIAL: return ks_launch<TM, TN, R, MODE, EPI_PARTIAL, KH>(g, s);
        default: return hipErrorInvalidValue;
    }
}

template <int TM, int TN, int R, bool CONV, int MODE = MODE_COOP>
hipError_t conv_epi(GemmGroup &g, int epi, hipStream_t s) {
    switch (epi) {
        case EPI_STORE_F32: return ks_launch<TM, TN, R, MODE, EPI_STORE_F32, 1, CONV>(g, s);
        case EPI_STORE_BF16: return ks_launch<TM, TN, R, MODE, EPI_STORE_BF16, 1, CONV>(g, s);
        case EPI_SWIGLU_F32: return ks_launch<TM, TN, R, MODE, EPI_SWIGLU_F32, 1, CONV>(g, s);
        case EPI_SWIGLU_BF16: return ks_launch<TM, TN, R, MODE, EPI_SWIGLU_BF16, 1, CONV>(g, s);
        case EPI_PARTIAL: return ks_launch<TM, TN, R, MODE, EPI_PARTIAL, 1, CONV>(g, s);
        case EPI_F32X:
            if constexpr (MODE == MODE_COOP64) return ks_launch<TM, TN, R, MODE, EPI_F32X, 1, CONV>(g, s);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_gemm_coop(GemmGroup &g, int epi, hipStream_t s) {
    if (g.nprob < 1 || g.nprob > 2) return hipErrorInvalidValue;
    const bool conv = g.p[0].conv_ic != 0;
    int64_t tiles = 0, tiles128 = 0;   // 128 x 64 and 128 x 128 tiles (64 output features for SwiGLU)
    for (int i = 0; i < g.nprob; ++i) {
        const GemmProblem &p = g.p[i];
        if (p.M < 16 || p.M % 16 || p.N < 1 || p.K < 32 || p.K % 32 || p.splits < 1 || (p.conv_ic != 0) != conv)
            return hipErrorInvalidValue;
        // split-K (slices [split][N][ld_y] of f32 partial sums) only as EPI_PARTIAL
        if (p.splits != 1 && (epi != EPI_PARTIAL || (p.K / 32) % p.splits)) return hipErrorInvalidValue;
        if (!p.w_tiled && (p.ld_w % 8 || ((uintptr_t) p.w & 15) || (p.w3 && ((uintptr_t) p.w3 & 15))))
            return hipErrorInvalidValue;
        if (p.w_tiled && epi_swiglu(epi)) return hipErrorInvalidValue;
        if (epi_swiglu(epi) && (!p.w3 || p.bias || p.M % 8)) return hipErrorInvalidValue;
        if (p.ld_x % 8 || ((uintptr_t) p.x & 15)) return hipErrorInvalidValue;
        if (epi == EPI_F32X && (p.M % 8 || p.ld_y % 8 || ((uintptr_t) p.y & 15) || (p.bias && ((uintptr_t) p.bias & 15)) ||
                                (p.accumulate && !p.y) ||
                                (p.snk_ea && (p.snk_period < 8 || p.snk_period % 8 || !p.snk_eb ||
                                              ((uintptr_t) p.snk_ea & 15) || ((uintptr_t) p.snk_eb & 15) ||
                                              ((uintptr_t) p.y2 & 15) || ((uintptr_t) p.yp & 15)))))
            return hipErrorInvalidValue;
        if (conv && (p.conv_ic % 32 || p.K % p.conv_ic || p.x_group_rows || p.conv_ow < 1 || p.conv_iw < 1 ||
                     p.conv_s < 1 || p.conv_d < 1 || p.conv_p < 0 || p.N % p.conv_ow || p.x_group_stride % 8))
            return hipErrorInvalidValue;
        tiles += (int64_t) ((p.M + (epi_swiglu(epi) ? 63 : 127)) / (epi_swiglu(epi) ? 64 : 128)) * ((p.N + 63) / 64) *
                 p.splits;
        tiles128 += (int64_t) ((p.M + (epi_swiglu(epi) ? 63 : 127)) / (epi_swiglu(epi) ? 64 : 128)) *
                    ((p.N + 127) / 128) * p.splits;
    }
    // Tile shape, measured on MI355X over the convolution / MLP / DiT shapes:
    // with K % 64 == 0 (and IC % 64 == 0 for convolutions) the 64-wide row
    // stages: 128 x 128 tiles (2 stages, two workgroups per CU) from ~400 such
    // tiles (the reference graph's 30 s convMLP w1 / w3, 1292 x 3072 x 2 x
    // 2816: 78 -> 52 us, half the operand loads per MFMA of 128 x 64 tiles
    // and one round of workgroups instead of two), 128 x 64 tiles (2 stages)
    // from ~400 of those, 64 x 64 tiles (3 stages) below; otherwise the
    // 32-wide stages, 128 x 64 from ~512 tiles. Tuning::coop_cfg forces a
    // shape (12, 22, 28, 29, 30, 32).
    bool k64 = true;
    for (int i = 0; i < g.nprob; ++i) k64 = k64 && g.p[i].K % 64 == 0 && (!conv || g.p[i].conv_ic % 64 == 0);
    int cfg = k64 ? (tiles128 >= 400 ? 32 : tiles >= 400 ? 29 : 30) : (tiles >= 512 ? 12 : 22);
    if (tuning().coop_cfg) cfg = tuning().coop_cfg;
    if (!k64 && cfg >= 28) cfg = tiles >= 512 ? 12 : 22;
    switch (cfg) {
        case 12: return conv ? conv_epi<8, 4, 4, true>(g, epi, s) : conv_epi<8, 4, 4, false>(g, epi, s);
        case 22: return conv ? conv_epi<4, 4, 4, true>(g, epi, s) : conv_epi<4, 4, 4, false>(g, epi, s);
        case 28: return conv ? conv_epi<8, 4, 3, true, MODE_COOP64>(g, epi, s) : conv_epi<8, 4, 3, false, MODE_COOP64>(g, epi, s);
        case 29: return conv ? conv_epi<8, 4, 2, true, MODE_COOP64>(g, epi, s) : conv_epi<8, 4, 2, false, MODE_COOP64>(g, epi, s);
        case 30: return conv ? conv_epi<4, 4, 3, true, MODE_COOP64>(g, epi, s) : conv_epi<4, 4, 3, false, MODE_COOP64>(g, epi, s);
        case 32: return conv ? conv_epi<8, 8, 2, true, MODE_COOP64>(g, epi, s) : conv_epi<8, 8, 2, false, MODE_COOP64>(g, epi, s);
        default: return hipErrorInvalidValue;
    }
}

int gemm_ks_bm(int cfg) {
    if (!cfg) cfg = 30;
    return cfg == 2 || cfg == 3 || cfg == 5 || cfg == 6 || cfg == 8 || cfg == 13 || cfg == 18 || cfg == 22 ||
                   cfg == 23 || cfg == 25 || cfg == 30 || cfg == 31 || cfg == 33 || cfg == 34 || cfg == 35 ||
                   cfg == 39 || cfg == 40
               ? 64
               : 128;
}

int gemm_ks_tiles(const GemmGroup &g, int bm, int bn) {
    int n = 0;
    for (int i = 0; i < g.nprob; ++i) {
        const GemmProblem &p = g.p[i];
        n = ((n + 7) & ~7) + ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn) * max(p.splits, 1);
    }
    return n;
}

hipError_t launch_gemm_ks(GemmGroup &g, int epi, int cfg, hipStream_t s) {
    if (g.nprob < 1 || g.nprob > 2) return hipErrorInvalidValue;
    for (int i = 0; i < g.nprob; ++i) {
        const GemmProblem &p = g.p[i];
        if (p.M < 16 || p.M % 16 || p.N < 1 || p.K < 32 || p.K % 32 || p.splits < 1 || p.splits > p.K / 32)
            return hipErrorInvalidValue;
        // row-major weights (the reference graph's qkv) as in launch_gemm_coop
        if (!p.w_tiled && (p.ld_w % 8 || ((uintptr_t) p.w & 15) || p.w3)) return hipErrorInvalidValue;
        if (epi != EPI_PARTIAL && p.splits != 1) return hipErrorInvalidValue;
        if (epi == EPI_QKV && (p.M % 192 || p.seq < 1 || (p.rope && !p.rope_cs))) return hipErrorInvalidValue;
    }
    // The DiT driver picks one of cfg 22 / 28 / 29 / 30 per projection (0:
    // 64 x 64 tiles of 64-wide row stages). The other tile shapes and main
    // loops (K-split rings, register prefetch, pipelined cooperative, 128 x
    // 128) exist for sweeps only and are compiled with TSK_SWEEP_VARIANTS.
    if (!cfg) cfg = 30;
#if TSK_SWEEP_VARIANTS
    if (cfg >= 6 && cfg <= 10) {
        // register prefetch: every wave's stage count a multiple of the depth
        const int depth = cfg == 7 || cfg == 8 || cfg == 10 ? 2 : 4;
        for (int i = 0; i < g.nprob; ++i) {
            const GemmProblem &p = g.p[i];
            const int kts = (p.K / 32 + p.splits - 1) / p.splits;
            if (kts % (4 * depth) || (p.K / 32) % p.splits) return hipErrorInvalidValue;
        }
    }
#endif
    for (int i = 0; i < g.nprob; ++i)
        if (g.p[i].M % gemm_ks_bm(cfg) && epi == EPI_QKV) return hipErrorInvalidValue;
    switch (cfg) {
        case 22: return ks_epi<4, 4, 4, MODE_COOP>(g, epi, s);    // 64 x 64 cooperative, 4 stages
        case 28: return ks_epi<8, 4, 3, MODE_COOP64>(g, epi, s);   // 128 x 64 cooperative, 3 stages of 64 k rows
        case 29: return ks_epi<8, 4, 2, MODE_COOP64>(g, epi, s);   // 128 x 64 cooperative, 2 stages of 64 k rows
        case 30: return ks_epi<4, 4, 3, MODE_COOP64>(g, epi, s);   // 64 x 64 cooperative, 3 stages of 64 k rows
#if TSK_SWEEP_VARIANTS
        case 1: return ks_epi<8, 4, 3>(g, epi, s);   // 128 x 64, 3 stages
        case 2: return ks_epi<4, 4, 3>(g, epi, s);   // 64 x 64, 3 stages
        case 3: return ks_epi<4, 8, 2>(g, epi, s);   // 64 x 128, 2 stages
        case 4: return ks_epi<8, 4, 2>(g, epi, s);   // 128 x 64, 2 stages
        case 5: return ks_epi<4, 4, 4>(g, epi, s);   // 64 x 64, 4 stages
        case 6: return ks_epi<4, 4, 4, MODE_DIRECT>(g, epi, s);   // 64 x 64, register prefetch 4 stages
        case 7: return ks_epi<8, 4, 2, MODE_DIRECT>(g, epi, s);   // 128 x 64, register prefetch 2 stages
        case 8: return ks_epi<4, 4, 2, MODE_DIRECT>(g, epi, s);   // 64 x 64, register prefetch 2 stages
        case 9: return ks_epi<8, 4, 4, MODE_DIRECT>(g, epi, s);   // 128 x 64, register prefetch 4 stages
        case 10: return ks_epi<8, 8, 2, MODE_DIRECT>(g, epi, s);  // 128 x 128, register prefetch 2 stages
        case 11: return ks_epi<8, 8, 4, MODE_COOP>(g, epi, s);    // 128 x 128 cooperative, 4 stages
        case 12: return ks_epi<8, 4, 4, MODE_COOP>(g, epi, s);    // 128 x 64 cooperative, 4 stages
        case 13: return ks_epi<4, 8, 4, MODE_COOP>(g, epi, s);    // 64 x 128 cooperative, 4 stages
        case 14: return ks_epi<8, 8, 3, MODE_COOP>(g, epi, s);    // 128 x 128 cooperative, 3 stages
        case 15: return ks_epi<8, 4, 3, MODE_COOP, 2>(g, epi, s); // 128 x 64 cooperative, 3 stages of 64 k
        case 16: return ks_epi<8, 4, 2, MODE_COOP, 2>(g, epi, s); // 128 x 64 cooperative, 2 stages of 64 k
        case 17: return ks_epi<8, 8, 2, MODE_COOP, 2>(g, epi, s); // 128 x 128 cooperative, 2 stages of 64 k
        case 18: return ks_epi<4, 8, 3, MODE_COOP, 2>(g, epi, s); // 64 x 128 cooperative, 3 stages of 64 k
        case 19: return ks_epi<8, 4, 6, MODE_COOP>(g, epi, s);    // 128 x 64 cooperative, 6 stages
        case 20: return ks_epi<8, 4, 3, MODE_COOP>(g, epi, s);    // 128 x 64 cooperative, 3 stages
        case 21: return ks_epi<8, 4, 2, MODE_COOP>(g, epi, s);    // 128 x 64 cooperative, 2 stages
        case 23: return ks_epi<4, 4, 3, MODE_COOP>(g, epi, s);    // 64 x 64 cooperative, 3 stages
        case 24: return ks_epi<8, 4, 4, MODE_COOP_PIPE>(g, epi, s);   // 128 x 64 cooperative, pipelined, 4 stages
        case 25: return ks_epi<4, 4, 4, MODE_COOP_PIPE>(g, epi, s);   // 64 x 64 cooperative, pipelined, 4 stages
        case 26: return ks_epi<8, 4, 5, MODE_COOP_PIPE>(g, epi, s);   // 128 x 64 cooperative, pipelined, 5 stages
        case 27: return ks_epi<8, 8, 4, MODE_COOP_PIPE>(g, epi, s);   // 128 x 128 cooperative, pipelined, 4 stages
        case 31: return ks_epi<4, 4, 2, MODE_COOP64>(g, epi, s);   // 64 x 64 cooperative, 2 stages of 64 k rows
        case 32: return ks_epi<8, 8, 2, MODE_COOP64>(g, epi, s);   // 128 x 128 cooperative, 2 stages of 64 k rows
        case 33: return ks_epi<4, 4, 4, MODE_COOP64>(g, epi, s);   // 64 x 64 cooperative, 4 stages of 64 k rows
        case 34: return ks_epi<4, 4, 5, MODE_COOP64>(g, epi, s);   // 64 x 64 cooperative, 5 stages of 64 k rows
        case 35: return ks_epi<4, 4, 6, MODE_COOP64>(g, epi, s);   // 64 x 64 cooperative, 6 stages of 64 k rows
        case 36: return ks_epi<8, 4, 2, MODE_PF>(g, epi, s);   // 128 x 64, 2 register stages, LDS double buffer
        case 37: return ks_epi<8, 4, 3, MODE_PF>(g, epi, s);   // 128 x 64, 3 register stages
        case 38: return ks_epi<8, 8, 2, MODE_PF>(g, epi, s);   // 128 x 128, 2 register stages
        case 39: return ks_epi<4, 4, 3, MODE_PF>(g, epi, s);   // 64 x 64, 3 register stages
        case 40: return ks_epi<4, 4, 4, MODE_PF>(g, epi, s);   // 64 x 64, 4 register stages
        case 41: return ks_epi<8, 4, 4, MODE_PF>(g, epi, s);   // 128 x 64, 4 register stages
        case 42: return ks_epi<8, 10, 3, MODE_COOP64>(g, epi, s);   // 128 x 160, 3 stages of 64 k rows
        case 43: return ks_epi<8, 10, 4, MODE_COOP64>(g, epi, s);   // 128 x 160, 4 stages
        case 44: return ks_epi<8, 12, 3, MODE_COOP64>(g, epi, s);   // 128 x 192, 3 stages
        case 45: return ks_epi<8, 10, 2, MODE_PF>(g, epi, s);       // 128 x 160, 2 register stages
        case 46: return ks_epi<8, 12, 2, MODE_PF>(g, epi, s);       // 128 x 192, 2 register stages
        case 47: return ks_epi<8, 10, 2, MODE_COOP64>(g, epi, s);   // 128 x 160, 2 stages
        case 48: return ks_epi<8, 12, 2, MODE_COOP64>(g, epi, s);   // 128 x 192, 2 stages
#endif
        default: return hipErrorInvalidValue;
    }
}

}  // namespace tsk
