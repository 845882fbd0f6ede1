// Dense GEMMs of the encoder layer on gfx950 MFMA:  C[M,N] = A[M,K] · B[N,K]ᵀ
// (+bias, activation, residual), the contraction of the reference's
// Kernel.MatMulT / MatMulTF16 (native/kernel.go:26-43) and MatMulTQ8
// (native/quant.go:99-137).  Both operands are K-contiguous (activations
// row-major, weights in nn.Linear [out,in] layout), exactly the reference's
// layout contract.
//
// f16 path: v_mfma_f32_16x16x32_f16, f32 accumulate.  i8 path:
// v_mfma_i32_16x16x64_i8, exact i32 accumulate, epilogue
// float(sum)·(sA·sB) + bias evaluated unfused as in quant.go:129-133.
//
// Tiling (template Cfg): BM×BN block tile, WM×WN waves each owning a
// (BM/WM)×(BN/WN) tile of 16×16 MFMA tiles, 128-byte K slices (64 f16 or
// 128 i8) staged through double-buffered LDS with one barrier per slice;
// the next slice's global loads are in flight while the current one is
// multiplied.  The MFMA is issued with the weight fragment as the A
// operand, so each lane ends up holding four consecutive output columns of
// one row: epilogue stores are 8/16-byte vectors, and the SwiGLU up/gate
// pair (interleaved in 16-row blocks at load) lands in the same lane.
#include <cstdlib>

#include "fh_common.h"
#include "gemm_epi.h"

namespace {
using namespace fh_epi;

constexpr int KFULL_BYTES = 128;  // K (in bytes) multiple every full-slice configuration divides

// KB: bytes of K per slice; PAD: bytes appended to each LDS row (the row
// stride decides the ds_read_b128 bank pattern: 160 bytes reads 16 rows at
// one offset without conflicts); PF: register prefetch depth in slices.
template <int BM_, int BN_, int WM_, int WN_, int PAD_, int PF_>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, PF = PF_, KB = 128;
    static constexpr int CPR = KB / 16;  // 16-byte chunks per slice row
    static constexpr int ROW = KB + PAD_;
    static constexpr int NT = 64 * WM * WN;
    static constexpr int MT = BM / WM / 16;  // 16-row MFMA tiles per wave
    static constexpr int NTL = BN / WN / 16; // 16-col MFMA tiles per wave
    static constexpr int ACH = BM * CPR / NT;  // 16-byte A chunks per thread per slice
    static constexpr int BCH = BN * CPR / NT;
    static_assert(ACH * NT == BM * CPR && BCH * NT == BN * CPR, "tile/thread mismatch");
    // The staged epilogue (32 rows per wave) fits in the operand LDS; small
    // tiles store straight from registers.
    static constexpr bool STAGE = (NT / 64) * 32 * (NTL * 16 * 4 + 16) <= 2 * BM * ROW;
};

// Workgroup barrier that orders LDS only.  __syncthreads() also fences
// global memory, which makes every barrier wait for all in-flight global
// loads and so cancels the prefetch of the next slices; the K loop only
// needs this wave's LDS reads and writes complete before the barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Maps the hardware block id onto (m-tile, n-tile) so that each of the 8
// XCDs (which receive block ids round-robin) works on a contiguous range of
// M tiles: an A row-panel is then fetched into one XCD's L2, not eight.
__device__ __forceinline__ void tile_coords(int &mt, int &nt) {
    const int gx = gridDim.x, nb = gridDim.x * gridDim.y;
    const int pid = blockIdx.y * gx + blockIdx.x;
    const int xcd = pid & 7, idx = pid >> 3;
    const int q = nb >> 3, r = nb & 7;
    const int logical = xcd * q + min(xcd, r) + idx;
    mt = logical / gx;
    nt = logical - mt * gx;
}

// rs: (mean, rstd) of A's row (LN_IN) or of the residual's row (RES_LN).
template <int ACT, bool OUT_F32, int LNM>
__device__ __forceinline__ void epilogue_store(const GemmArgs &g, int row, int col, f32x4 v,
                                               f32x4 gate, f32x2 rs) {
    if (LNM == fh::LN_IN) {
        v = ln_fold(g, col, v, rs);
        if (ACT == fh::ACT_SWIGLU) gate = ln_fold(g, col + 16, gate, rs);
    }
    if (ACT == fh::ACT_SWIGLU) {
        // col is the packed up-column; output column folds the 16-row interleave.
        const int ocol = ((col >> 5) << 4) + (col & 15);
        if (g.bias) {
            v += *(const f32x4 *)(g.bias + col);
            gate += *(const f32x4 *)(g.bias + col + 16);
        }
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = v[i] * silu(gate[i]);
        if (OUT_F32) {
            *(f32x4 *)((float *)g.C + (size_t)row * g.ldc + ocol) = o;
        } else {
            f16x4 h = {to_f16(o[0]), to_f16(o[1]), to_f16(o[2]), to_f16(o[3])};
            *(f16x4 *)((f16 *)g.C + (size_t)row * g.ldc + ocol) = h;
        }
        return;
    }
    if (g.bias) v += *(const f32x4 *)(g.bias + col);
    if (ACT == fh::ACT_GELU) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = gelu_erf(v[i]);
    }
    const size_t rrow = g.res_map ? (size_t)g.res_map[row] : (size_t)row;
    if (g.resid) {
        v += *(const f32x4 *)(g.resid + rrow * g.ldr + col);
    } else if (g.resid_h) {
        const f16x4 r = *(const f16x4 *)(g.resid_h + rrow * g.ldr + col);
        if (LNM == fh::RES_LN) v += ln_resid(g, rs, col, r);
        else v += (f32x4){(float)r[0], (float)r[1], (float)r[2], (float)r[3]};
    }
    if (OUT_F32) {
        *(f32x4 *)((float *)g.C + (size_t)row * g.ldc + col) = v;
    } else {
        f16x4 h = {to_f16(v[0]), to_f16(v[1]), to_f16(v[2]), to_f16(v[3])};
        *(f16x4 *)((f16 *)g.C + (size_t)row * g.ldc + col) = h;
    }
}

// Epilogue over a wave's tiles.  Lane holds C[row][col .. col+3] for
// row = tile_m + lane%16, col = tile_n + (lane/16)·4.
template <class C, bool I8, int ACT, bool OUT_F32, int LNM>
__device__ __forceinline__ void store_tiles(const GemmArgs &g, int m0, int n0, int wm, int wn, int lane,
                                            const f32x4 (&acc)[C::NTL][C::MT], const i32x4 (&iacc)[C::NTL][C::MT]) {
#pragma unroll
    for (int tm = 0; tm < C::MT; ++tm) {
        const int rl = (wm * C::MT + tm) * 16 + (lane & 15);
        const int row = m0 + rl;
        if (row >= g.M) continue;
        const f32x2 rs = LNM == fh::RES_LN  ? g.stats_in[g.res_map ? g.res_map[row] : row]
                         : LNM == fh::LN_IN ? g.stats_in[row]
                                            : (f32x2){0.f, 0.f};
        float sa = 0.f;
        if (I8) sa = g.a_scale[row];
#pragma unroll
        for (int tn = 0; tn < C::NTL; ++tn) {
            if (ACT == fh::ACT_SWIGLU && (tn & 1)) continue;
            const int col = n0 + (wn * C::NTL + tn) * 16 + (lane >> 4) * 4;
            if (col >= g.N) continue;
            f32x4 v, gate = {0.f, 0.f, 0.f, 0.f};
            if (I8) {
                const f32x4 sb = *(const f32x4 *)(g.b_scale + col);
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = __fmul_rn((float)iacc[tn][tm][i], __fmul_rn(sa, sb[i]));
                if (ACT == fh::ACT_SWIGLU) {
                    const f32x4 sg = *(const f32x4 *)(g.b_scale + col + 16);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        gate[i] = __fmul_rn((float)iacc[tn + 1][tm][i], __fmul_rn(sa, sg[i]));
                }
            } else {
                v = acc[tn][tm];
                if (ACT == fh::ACT_SWIGLU) gate = acc[tn + 1][tm];
            }
            epilogue_store<ACT, OUT_F32, LNM>(g, row, col, v, gate, rs);
        }
    }
}

// Epilogue through LDS.  A lane's MFMA results are four columns of one row,
// so storing them directly writes 16 rows × 32 bytes per instruction.  Here
// each wave stages 32 rows of its (after bias/activation/scales) tile in its
// own LDS region, then writes whole row segments with 16-byte stores, adding
// the residual in the same coalesced pass.  Needs whole block columns (N a
// multiple of BN: the launcher checks), a multiple of 32 columns per wave and
// the operand LDS free (after the K loop's last barrier).
template <class C, bool I8, int ACT, bool OUT_F32, int LNM>
__device__ __forceinline__ void store_tiles_lds(const GemmArgs &g, int m0, int n0, int wm, int wn, int lane,
                                                int wave, const f32x4 (&acc)[C::NTL][C::MT],
                                                const i32x4 (&iacc)[C::NTL][C::MT], uint8_t *lds) {
    static_assert(C::MT % 2 == 0 && C::NTL % 2 == 0, "staged epilogue works on 32-row, 32-column multiples");
    constexpr int WTN = C::NTL * 16;                           // wave tile width
    constexpr int OC = ACT == fh::ACT_SWIGLU ? WTN / 2 : WTN;  // output columns per wave
    constexpr bool R16 = ACT == fh::ACT_RES16;
    constexpr int ESZ = (OUT_F32 || R16) ? 4 : 2;        // staged element size (bytes)
    constexpr int RS = OC * ESZ + 16;                    // LDS row stride (bytes)
    constexpr int CPR = OC * ESZ / 16;                   // 16-byte chunks per row
    uint8_t *region = lds + wave * 32 * RS;
    const int ocol0 = ACT == fh::ACT_SWIGLU ? (n0 + wn * WTN) >> 1 : n0 + wn * WTN;
#pragma unroll
    for (int p = 0; p < C::MT / 2; ++p) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int tm = 2 * p + h;
            const int rl = (wm * C::MT + tm) * 16 + (lane & 15);
            const int row = m0 + rl;
            const f32x2 rs = LNM == fh::LN_IN ? g.stats_in[min(row, g.M - 1)] : (f32x2){0.f, 0.f};
            float sa = 0.f;
            if (I8) sa = g.a_scale[min(row, g.M - 1)];
#pragma unroll
            for (int tn = 0; tn < C::NTL; ++tn) {
                if (ACT == fh::ACT_SWIGLU && (tn & 1)) continue;
                const int col = n0 + (wn * C::NTL + tn) * 16 + (lane >> 4) * 4;
                f32x4 v, gate = {0.f, 0.f, 0.f, 0.f};
                if (I8) {
                    const f32x4 sb = *(const f32x4 *)(g.b_scale + col);
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = __fmul_rn((float)iacc[tn][tm][i], __fmul_rn(sa, sb[i]));
                    if (ACT == fh::ACT_SWIGLU) {
                        const f32x4 sg = *(const f32x4 *)(g.b_scale + col + 16);
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            gate[i] = __fmul_rn((float)iacc[tn + 1][tm][i], __fmul_rn(sa, sg[i]));
                    }
                } else {
                    v = acc[tn][tm];
                    if (ACT == fh::ACT_SWIGLU) gate = acc[tn + 1][tm];
                }
                if (LNM == fh::LN_IN) {
                    v = ln_fold(g, col, v, rs);
                    if (ACT == fh::ACT_SWIGLU) gate = ln_fold(g, col + 16, gate, rs);
                }
                if (ACT == fh::ACT_SWIGLU) {
                    if (g.bias) {
                        v += *(const f32x4 *)(g.bias + col);
                        gate += *(const f32x4 *)(g.bias + col + 16);
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = v[i] * silu(gate[i]);
                } else {
                    if (g.bias) v += *(const f32x4 *)(g.bias + col);
                    if (ACT == fh::ACT_GELU) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) v[i] = gelu_erf(v[i]);
                    }
                }
                const int lc = (ACT == fh::ACT_SWIGLU ? (tn >> 1) : tn) * 16 + (lane >> 4) * 4;
                uint8_t *dst = region + (h * 16 + (lane & 15)) * RS + lc * ESZ;
                if (OUT_F32 || R16) {
                    *(f32x4 *)dst = v;
                } else {
                    *(f16x4 *)dst = (f16x4){to_f16(v[0]), to_f16(v[1]), to_f16(v[2]), to_f16(v[3])};
                }
            }
        }
        if (R16) {
            // 8 output columns per lane step: two staged f32 chunks plus the
            // binary16 residual, rounded once, one 16-byte store.
            constexpr int C8 = OC / 8;  // 8-column output chunks per row
            static_assert((32 * C8) % 64 == 0, "whole lane steps");
#pragma unroll
            for (int j = 0; j < 32 * C8 / 64; ++j) {
                const int c = lane + 64 * j, r = c / C8, ch = c % C8;
                const int grow = m0 + (wm * C::MT + 2 * p) * 16 + r;
                const f32x4 lo = *(const f32x4 *)(region + r * RS + ch * 32);
                const f32x4 hi = *(const f32x4 *)(region + r * RS + ch * 32 + 16);
                if (grow >= g.M) continue;
                const int gcol = ocol0 + ch * 8;
                f32x4 r0 = {0.f, 0.f, 0.f, 0.f}, r1 = r0;
                if (g.resid_h) {
                    const int rgrow = g.res_map ? g.res_map[grow] : grow;
                    const f16x8 rr = *(const f16x8 *)(g.resid_h + (size_t)rgrow * g.ldr + gcol);
                    const f16x4 ra = {rr[0], rr[1], rr[2], rr[3]}, rb = {rr[4], rr[5], rr[6], rr[7]};
                    if (LNM == fh::RES_LN) {
                        const f32x2 st = g.stats_in[rgrow];
                        r0 = ln_resid(g, st, gcol, ra);
                        r1 = ln_resid(g, st, gcol + 4, rb);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            r0[i] = (float)ra[i];
                            r1[i] = (float)rb[i];
                        }
                    }
                }
                f16x8 o;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    o[i] = to_f16(lo[i] + r0[i]);
                    o[4 + i] = to_f16(hi[i] + r1[i]);
                }
                *(f16x8 *)((f16 *)g.C + (size_t)grow * g.ldc + gcol) = o;
            }
            continue;
        }
        // Same-wave LDS accesses complete in order: the rows are readable now.
        static_assert((32 * CPR) % 64 == 0, "whole lane steps");
#pragma unroll
        for (int j = 0; j < 32 * CPR / 64; ++j) {
            const int c = lane + 64 * j, r = c / CPR, ch = c % CPR;
            const int grow = m0 + (wm * C::MT + 2 * p) * 16 + r;
            i32x4 d = *(const i32x4 *)(region + r * RS + ch * 16);
            if (grow >= g.M) continue;
            const int gcol = ocol0 + ch * (16 / ESZ);
            if (OUT_F32 && (g.resid || g.resid_h)) {
                f32x4 v = __builtin_bit_cast(f32x4, d);
                const size_t rgrow = g.res_map ? (size_t)g.res_map[grow] : (size_t)grow;
                if (g.resid) {
                    v += *(const f32x4 *)(g.resid + rgrow * g.ldr + gcol);
                } else {
                    const f16x4 rr = *(const f16x4 *)(g.resid_h + rgrow * g.ldr + gcol);
                    v += (f32x4){(float)rr[0], (float)rr[1], (float)rr[2], (float)rr[3]};
                }
                d = __builtin_bit_cast(i32x4, v);
            }
            *(i32x4 *)((uint8_t *)g.C + ((size_t)grow * g.ldc + gcol) * ESZ) = d;
        }
    }
}

// amdgpu_waves_per_eu(1): one block of 2–8 waves fills a CU's LDS anyway, so
// the scheduler may trade occupancy for instruction-level parallelism.
template <class C, bool I8, bool KFULL, int ACT, bool OUT_F32, int LNM>
__global__ __launch_bounds__(C::NT) __attribute__((amdgpu_waves_per_eu(1))) void gemm_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) uint8_t As[2][C::BM * C::ROW];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[2][C::BN * C::ROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / C::WN, wn = wave % C::WN;
    int mt, nt;
    tile_coords(mt, nt);
    const int m0 = mt * C::BM, n0 = nt * C::BN;
    constexpr int ESZ = I8 ? 1 : 2;
    const int kbytes = g.K * ESZ;
    const uint8_t *A = (const uint8_t *)g.A;
    const uint8_t *B = (const uint8_t *)g.B;
    const size_t lda = (size_t)g.lda * ESZ, ldb = (size_t)g.ldb * ESZ;
    const i32x4 zero = {0, 0, 0, 0};

    // Per-thread source rows (clamped into the matrix; clamped rows are
    // computed and never stored) for chunk c = tid + i·NT: row c/8, bytes (c%8)·16.
    const uint8_t *asrc[C::ACH];
    const uint8_t *bsrc[C::BCH];
#pragma unroll
    for (int i = 0; i < C::ACH; ++i) {
        const int c = tid + i * C::NT;
        asrc[i] = A + (size_t)min(m0 + c / C::CPR, g.M - 1) * lda + (c % C::CPR) * 16;
    }
#pragma unroll
    for (int i = 0; i < C::BCH; ++i) {
        const int c = tid + i * C::NT;
        bsrc[i] = B + (size_t)min(n0 + c / C::CPR, g.N - 1) * ldb + (c % C::CPR) * 16;
    }

    // Two register stages: slice k+2 is fetched while slice k is multiplied
    // and slice k+1 waits in registers, so ~two slices of MFMA work cover the
    // global-load latency.
    i32x4 ra[C::PF][C::ACH], rb[C::PF][C::BCH];
    auto gload = [&](int st, int kb0) {
#pragma unroll
        for (int i = 0; i < C::ACH; ++i) {
            if (KFULL) {
                ra[st][i] = *(const i32x4 *)(asrc[i] + kb0);
            } else {
                const int kb = kb0 + ((tid + i * C::NT) % C::CPR) * 16;
                ra[st][i] = kb < kbytes ? *(const i32x4 *)(asrc[i] + kb0) : zero;
            }
        }
#pragma unroll
        for (int i = 0; i < C::BCH; ++i) {
            if (KFULL) {
                rb[st][i] = *(const i32x4 *)(bsrc[i] + kb0);
            } else {
                const int kb = kb0 + ((tid + i * C::NT) % C::CPR) * 16;
                rb[st][i] = kb < kbytes ? *(const i32x4 *)(bsrc[i] + kb0) : zero;
            }
        }
    };
    auto sstore = [&](int st, int buf) {
#pragma unroll
        for (int i = 0; i < C::ACH; ++i) {
            const int c = tid + i * C::NT;
            *(i32x4 *)&As[buf][(c / C::CPR) * C::ROW + (c % C::CPR) * 16] = ra[st][i];
        }
#pragma unroll
        for (int i = 0; i < C::BCH; ++i) {
            const int c = tid + i * C::NT;
            *(i32x4 *)&Bs[buf][(c / C::CPR) * C::ROW + (c % C::CPR) * 16] = rb[st][i];
        }
    };

    f32x4 acc[C::NTL][C::MT];
    i32x4 iacc[C::NTL][C::MT];
#pragma unroll
    for (int a = 0; a < C::NTL; ++a)
#pragma unroll
        for (int b = 0; b < C::MT; ++b) {
            acc[a][b] = (f32x4){0.f, 0.f, 0.f, 0.f};
            iacc[a][b] = zero;
        }

    constexpr int KB = C::KB;
    const int nk = (kbytes + KB - 1) / KB;
    const int arow0 = (wm * C::MT * 16 + (lane & 15)) * C::ROW + (lane >> 4) * 16;
    const int brow0 = (wn * C::NTL * 16 + (lane & 15)) * C::ROW + (lane >> 4) * 16;
    auto compute = [&](int cur) {
#pragma unroll
        for (int kk = 0; kk < KB; kk += 64) {  // 64 bytes of K per MFMA step
            i32x4 af[C::MT], bf[C::NTL];
#pragma unroll
            for (int t = 0; t < C::MT; ++t) af[t] = *(const i32x4 *)&As[cur][arow0 + t * 16 * C::ROW + kk];
#pragma unroll
            for (int t = 0; t < C::NTL; ++t) bf[t] = *(const i32x4 *)&Bs[cur][brow0 + t * 16 * C::ROW + kk];
#pragma unroll
            for (int tn = 0; tn < C::NTL; ++tn)
#pragma unroll
                for (int tm = 0; tm < C::MT; ++tm) {
                    if (I8) {
                        iacc[tn][tm] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[tn], af[tm], iacc[tn][tm], 0, 0, 0);
                    } else {
                        acc[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(f16x8, bf[tn]), __builtin_bit_cast(f16x8, af[tm]), acc[tn][tm], 0,
                            0, 0);
                    }
                }
        }
    };
    // Loads and stores in the loop are unconditional (the slice index is
    // clamped, so the last iterations re-fetch the final slice into a buffer
    // nobody reads again): a conditional load would make the compiler's
    // counter merge at the join wait for every outstanding load.
    const int last = (nk - 1) * KB;
    if (C::PF == 1) {
        // One register stage: slice kt+1 is fetched while slice kt is multiplied.
        gload(0, 0);
        sstore(0, 0);
        lds_barrier();
        for (int kt = 0; kt < nk; ++kt) {
            gload(0, min((kt + 1) * KB, last));
            __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the MFMAs
            compute(kt & 1);
            __builtin_amdgcn_sched_barrier(0);
            sstore(0, (kt + 1) & 1);
            lds_barrier();
        }
    } else {
        // Two register stages; slice kt lives in LDS buffer kt%2 and, before
        // that, in register stage kt%2.
        auto step = [&](int kt, int par) {
            gload(par, min((kt + 2) * KB, last));  // stage par was stored last iteration
            __builtin_amdgcn_sched_barrier(0);     // keep the prefetch ahead of the MFMAs
            compute(par);
            __builtin_amdgcn_sched_barrier(0);
            sstore(par ^ 1, par ^ 1);
            lds_barrier();
        };
        gload(0, 0);
        gload(1, min(KB, last));
        sstore(0, 0);
        lds_barrier();
        int kt = 0;
        for (; kt + 1 < nk; kt += 2) {
            step(kt, 0);
            step(kt + 1, 1);
        }
        if (kt < nk) step(kt, 0);
    }

    // The staged epilogue reuses the A stages.
    if constexpr (C::STAGE) {
        if (KFULL && g.epi_lds) {
            store_tiles_lds<C, I8, ACT, OUT_F32, LNM>(g, m0, n0, wm, wn, lane, wave, acc, iacc, &As[0][0]);
            return;
        }
    }
    store_tiles<C, I8, ACT, OUT_F32, LNM>(g, m0, n0, wm, wn, lane, acc, iacc);
}

// Tile configurations (block tile, wave grid, row pad, prefetch depth).
using C0 = Cfg<128, 128, 2, 2, 16, 1>;
using C1 = Cfg<128, 128, 2, 2, 32, 1>;
using C2 = Cfg<256, 128, 4, 2, 32, 1>;
using C3 = Cfg<256, 128, 4, 2, 32, 2>;
using C5 = Cfg<256, 256, 2, 4, 32, 1>;
using C6 = Cfg<64, 64, 2, 2, 16, 2>;

template <class C, bool I8, bool KFULL, int ACT, bool OUT_F32, int LNM>
void launch_one(const GemmArgs &g, hipStream_t s) {
    dim3 grid((g.N + C::BN - 1) / C::BN, (g.M + C::BM - 1) / C::BM);
    hipLaunchKernelGGL((gemm_kernel<C, I8, KFULL, ACT, OUT_F32, LNM>), grid, dim3(C::NT), 0, s, g);
}

template <class C, bool I8, bool KFULL>
hipError_t launch_cfg(const GemmArgs &ga, int act, bool out_f32, int ln, hipStream_t s) {
    GemmArgs g = ga;
    g.epi_lds = g.epi_lds && g.N % C::BN == 0;  // the staged epilogue writes whole block columns
    if (ln != fh::LN_NONE) {  // binary16 only
        if constexpr (I8) {
            return hipErrorInvalidValue;
        } else if (ln == fh::LN_IN && KFULL && !out_f32) {
            if (act == fh::ACT_NONE) launch_one<C, false, KFULL, fh::ACT_NONE, false, fh::LN_IN>(g, s);
            else if (act == fh::ACT_GELU) launch_one<C, false, KFULL, fh::ACT_GELU, false, fh::LN_IN>(g, s);
            else if (act == fh::ACT_SWIGLU) launch_one<C, false, KFULL, fh::ACT_SWIGLU, false, fh::LN_IN>(g, s);
            else return hipErrorInvalidValue;
        } else if (ln == fh::RES_LN && !out_f32 && act == fh::ACT_RES16) {
            launch_one<C, false, KFULL, fh::ACT_RES16, false, fh::RES_LN>(g, s);
        } else {
            return hipErrorInvalidValue;
        }
    } else if (act == fh::ACT_NONE) {
        if (out_f32) launch_one<C, I8, KFULL, fh::ACT_NONE, true, fh::LN_NONE>(g, s);
        else launch_one<C, I8, KFULL, fh::ACT_NONE, false, fh::LN_NONE>(g, s);
    } else if (act == fh::ACT_GELU) {
        if (out_f32) launch_one<C, I8, KFULL, fh::ACT_GELU, true, fh::LN_NONE>(g, s);
        else launch_one<C, I8, KFULL, fh::ACT_GELU, false, fh::LN_NONE>(g, s);
    } else if (act == fh::ACT_SWIGLU) {
        if (out_f32) launch_one<C, I8, KFULL, fh::ACT_SWIGLU, true, fh::LN_NONE>(g, s);
        else launch_one<C, I8, KFULL, fh::ACT_SWIGLU, false, fh::LN_NONE>(g, s);
    } else if (act == fh::ACT_RES16 && !out_f32) {
        launch_one<C, I8, KFULL, fh::ACT_RES16, false, fh::LN_NONE>(g, s);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// FUTON_GEMM_TILE=0,1,2,3,5,6 pins a configuration (tuning knob); otherwise
// the choice depends only on the problem shape.
int forced_cfg() {
    static const int v = [] {
        const char *e = getenv("FUTON_GEMM_TILE");
        return e ? atoi(e) : -1;
    }();
    return v;
}

template <bool I8>
hipError_t launch(const GemmArgs &ga, int act, bool out_f32, int ln, hipStream_t s) {
    if (ga.M <= 0) return hipSuccess;
    GemmArgs g = ga;
    if (act == fh::ACT_NONE && !out_f32 && g.resid_h && !g.resid) act = fh::ACT_RES16;
    const int nout = act == fh::ACT_SWIGLU ? g.N / 2 : g.N;
    const bool has_res = g.resid || g.resid_h;
    g.epi_lds = (nout % (act == fh::ACT_SWIGLU ? 32 : 64) == 0) && (g.N % 64 == 0) &&
                (out_f32 || act == fh::ACT_RES16 || !has_res) && (g.ldc % 8 == 0) && (!has_res || g.ldr % 8 == 0);
    const bool kfull = (g.K * (I8 ? 1 : 2)) % KFULL_BYTES == 0;
    if (ln == fh::LN_IN && !kfull) return hipErrorInvalidValue;  // the LN_IN kernels are built for whole slices
    if (!kfull) return launch_cfg<C0, I8, false>(g, act, out_f32, ln, s);
    int cfg = forced_cfg();
    if (cfg < 0 || cfg > 6 || cfg == 4) {
        // 256×256 when it still gives every CU a block; 256×128 down to half
        // the CUs (it beats 128×128 on the N = H projections even there).
        // 64×64 when even 128×128 leaves most CUs idle (the few-row GEMMs of
        // the CLS-pooled last layer).
        const long m256 = (g.M + 255) / 256, m128 = (g.M + 127) / 128;
        if (g.N % 256 == 0 && m256 * (g.N / 256) >= 256) cfg = 5;
        else if (m256 * ((g.N + 127) / 128) >= 128) cfg = 3;
        else if (m128 * ((g.N + 127) / 128) >= 64) cfg = 0;
        else cfg = 6;
    }
    switch (cfg) {
    case 1: return launch_cfg<C1, I8, true>(g, act, out_f32, ln, s);
    case 2: return launch_cfg<C2, I8, true>(g, act, out_f32, ln, s);
    case 3: return launch_cfg<C3, I8, true>(g, act, out_f32, ln, s);
    case 5: return launch_cfg<C5, I8, true>(g, act, out_f32, ln, s);
    case 6: return launch_cfg<C6, I8, true>(g, act, out_f32, ln, s);
    default: return launch_cfg<C0, I8, true>(g, act, out_f32, ln, s);
    }
}

}  // namespace

namespace fh {
hipError_t gemm_f16(const GemmArgs &a, int act, bool out_f32, hipStream_t s, int ln) {
    return launch<false>(a, act, out_f32, ln, s);
}
hipError_t gemm_i8(const GemmArgs &a, int act, bool out_f32, hipStream_t s) {
    return launch<true>(a, act, out_f32, fh::LN_NONE, s);
}
}  // namespace fh
