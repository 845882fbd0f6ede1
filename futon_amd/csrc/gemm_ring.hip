// Persistent binary16 GEMM for the encoder's projections on gfx950:
// C[M,N] = A[M,K] · Bᵀ, the contraction of the reference's Kernel.MatMulTF16
// (native/kernel.go:26-43) with the same epilogues as gemm.hip (bias, GELU,
// residual, the folded-LayerNorm modes).
//
// Layout and schedule (the default configurations, R2 and R5 below; the
// others are tuning alternatives):
// * Two persistent 4-wave blocks per CU, each looping over 128×128 output
//   tiles (a wave owns 64×64), or, for GEMMs whose 256×256 tiles cover every
//   CU (the BERT-base-sized projections), one persistent 8-wave block per CU
//   over 256×256 tiles (a wave owns 128×64), which halves the operand bytes
//   streamed per MFMA.  Each of the 8 XCDs owns a contiguous range of
//   tiles, so an A row panel is fetched into one XCD's L2 and reused there
//   by all of that panel's column tiles.
// * Operands stream into a 2-slot LDS ring (32 or 64 KB per 64-wide K slice
//   per block) straight from global memory with buffer_load … lds (no VGPR
//   staging, no LDS store instructions).  The ring runs across tile
//   boundaries: the next tile's first slice is in flight during the current
//   tile's last slice and its epilogue, and while one block waits at its
//   barrier the other keeps the matrix cores busy.  Rows past M read as zero
//   through the buffer range check.
// * LDS rows are 128 bytes with the 16-byte chunk index XOR-ed with row%8,
//   which makes the MFMA fragment reads (16 rows × one chunk) conflict-free.
// * v_mfma_f32_16x16x32_f16 with the weight fragment as the A operand: a
//   lane holds four consecutive MFMA rows of one token.  The weights are
//   stored permuted within each 64-row block (ring_pack_row) so that those
//   MFMA rows are output features g·8 + {0..7} (+32), and every lane writes
//   two whole 16-byte runs of 8 features: coalesced stores straight from
//   registers, no LDS staging.
// The accumulation order over K is the one gemm.hip uses (same slices, same
// MFMA shape) and the epilogue arithmetic is shared, so both kernels give the
// same bits for the same operands.
#include <cstdlib>

#include "fh_common.h"
#include "gemm_epi.h"
#include "lds_dma.h"

namespace {
using namespace fh_epi;
using fh_dma::buf_rsrc;
using fh_dma::dma16;

// Ring configuration: BM×BN output tile, WM×WN waves, SLOTS ring slots;
// PERSIST: one block per CU looping over tiles (else one block per tile,
// the hardware scheduling them as CUs free up); ROWB: bytes of K per slice
// row (128: 64-wide K slices; 64: 32-wide, for deeper rings).
template <int BM_, int BN_, int WM_, int WN_, int SLOTS_, bool PERSIST_, int ROWB_ = 128>
struct RCfg {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, SLOTS = SLOTS_, ROWB = ROWB_;
    static constexpr bool PERSIST = PERSIST_;
    static constexpr int RPB = 1024 / ROWB;                // slot rows per 1-KB DMA block
    static constexpr int KS = ROWB / 64;                   // 32-wide MFMA k-steps per slice
    static constexpr int NT = 64 * WM * WN;                // threads
    static constexpr int MT = BM / WM / 16;                // token tiles per wave
    static constexpr int NTL = BN / WN / 16;               // feature tiles per wave (the 64-row packing block)
    static constexpr int STAGE = (BM + BN) * ROWB;         // bytes per ring slot
    static constexpr int DPW = (BM + BN) / RPB / (WM * WN);  // 1-KB DMA blocks per wave per slice
    static constexpr int BPC = 163840 / (SLOTS * STAGE);   // blocks per CU the LDS allows
    static_assert(NTL == 4 && DPW * RPB * WM * WN == BM + BN && BM % RPB == 0 && SLOTS >= 2 && BPC >= 1 &&
                      (ROWB == 128 || ROWB == 64),
                  "ring tile shape");
};
constexpr int BN = 128;     // every configuration's column tile (the packing unit × 2)

// {x of lane l, y of lane l} → {x, y} of lanes 0..31 and 32..63 exchanged
// between the halves: lanes < 32 get {x[l], x[l + 32]}, lanes ≥ 32
// {y[l − 32], y[l]} (v_permlane32_swap).  Operands and results pass through
// empty asm statements: this compiler can otherwise fold float arithmetic on
// the two results as if both were the first.
__device__ __forceinline__ f32x2 swap_halves(float x, float y) {
    unsigned a = __builtin_bit_cast(unsigned, x), b = __builtin_bit_cast(unsigned, y);
    asm volatile("" : "+v"(a), "+v"(b));
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    unsigned r0 = r[0], r1 = r[1];
    asm volatile("" : "+v"(r0), "+v"(r1));
    return (f32x2){__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1)};
}
constexpr int BM_MAX = 256;

// RES: no residual (0), f32 (1) or binary16 (2); BIAS: g.bias is set.  The
// epilogue is straight-line code for each combination, so the number of
// vector memory instructions it issues is a constant the ring's waits use.
// I8: A and B are int8 codes (v_mfma_i32_16x16x64_i8, exact i32 sums; a
// 128-byte slice row is 128 values), scaled in the epilogue by
// a_scale[row]·b_scale[col] as gemm.hip's int8 kernel does.
template <class R, int ACT, bool OUT_F32, int LNM, bool BIAS, int RES, bool I8 = false>
__global__ __launch_bounds__(R::NT) __attribute__((amdgpu_waves_per_eu(2))) void ring_kernel(GemmArgs g, int ntn,
                                                                                              int per_part, int cg) {
    constexpr int BM = R::BM, WN = R::WN, SLOTS = R::SLOTS;
    constexpr int MT = R::MT, NTL = R::NTL, STAGE = R::STAGE, DPW = R::DPW, BN = R::BN;
    constexpr int ROWB = R::ROWB, RPB = R::RPB, KS = R::KS;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[SLOTS * STAGE];
    static_assert(!I8 || (ACT != fh::ACT_SWIGLU && LNM == fh::LN_NONE && RES != 2), "int8 ring forms");

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;

    // This block's tiles: the column tiles are split into cg groups of
    // cols = ntn / cg, and XCD x (= block id mod 8) takes column group x % cg.
    // The group's tiles, numbered row-major (u = row·cols + column), are
    // split among its 8 / cg XCDs: XCD x owns [p·per_part, (p+1)·per_part)
    // with p = x / cg, and its blocks take them round-robin.
    const int nbx = gridDim.x >> 3, xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
    const int cols = ntn / cg, col0 = (xcd % cg) * cols, part = xcd / cg;
    const int ntiles = ((g.M + BM - 1) / BM) * cols;
    const int t0 = part * per_part + j, tend = min(ntiles, (part + 1) * per_part);
    const int ntile = t0 < tend ? (tend - t0 + nbx - 1) / nbx : 0;
    const int nk = g.K / (I8 ? ROWB : ROWB / 2);
    const int nsl = ntile * nk;  // slices this block multiplies
    if (nsl == 0) return;

    constexpr uint32_t EB = I8 ? 1 : 2;  // operand bytes per value
    const uint32_t lda_b = (uint32_t)g.lda * EB, ldb_b = (uint32_t)g.ldb * EB;
    const __amdgpu_buffer_rsrc_t rA = buf_rsrc(g.A, (uint32_t)g.M * lda_b);
    const __amdgpu_buffer_rsrc_t rB = buf_rsrc(g.B, (uint32_t)g.N * ldb_b);
    const uint32_t ring0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)ring;

    // DMA block b of a slot holds slot rows RPB·b .. RPB·b + RPB − 1 (rows
    // < BM: A, else B).  128-byte rows: lane l writes physical chunk l%8 of
    // row 8b + l/8, i.e. logical chunk (l%8) ^ (l/8).  64-byte rows: lane l
    // writes physical chunk l%4 of row 16b + l/4, logical chunk
    // (l%4) ^ ((l/16)%4).  Either way the 16 rows × one logical chunk that a
    // fragment read takes land on 16 distinct 16-byte bank groups.
    const uint32_t lrow = ROWB == 128 ? lane >> 3 : lane >> 2;
    const uint32_t lchunk = (ROWB == 128 ? (lane & 7) ^ (lane >> 3) : (lane & 3) ^ ((lane >> 4) & 3)) * 16;
    // Per DMA block of this wave (wave-uniform, fixed for the kernel): operand
    // and row offset inside the tile's operand rows.
    bool isA[DPW];
#pragma unroll
    for (int i = 0; i < DPW; ++i) isA[i] = (wave * DPW + i) * RPB < BM;
    // Issues the next slice of this block's sequence (past the end: the last
    // slice again, into a slot nobody reads) into the next slot.  Slices are
    // issued in order, so the slice's tile and K position advance by
    // counting, not by dividing: integer division is a long scalar sequence
    // that would delay the waves' matrix instructions every slice.
    int is_kk = 0, is_left = nsl, is_slot = 0, is_mt, is_nt;
    {
        is_mt = t0 / cols;
        is_nt = t0 - is_mt * cols;
    }
    auto issue = [&] {
        const int kk = is_kk, mt = is_mt, nt = col0 + is_nt;
        const uint32_t slot = ring0 + (uint32_t)is_slot * STAGE;
        is_slot = is_slot + 1 == SLOTS ? 0 : is_slot + 1;
        if (is_left > 1) {  // advance to the following slice (the last one is repeated)
            --is_left;
            if (++is_kk == nk) {
                is_kk = 0;
                is_nt += nbx;  // the next tile of this block: t + nbx
                while (is_nt >= cols) {
                    is_nt -= cols;
                    ++is_mt;
                }
            }
        }
        const uint32_t soff = (uint32_t)kk * ROWB;
        const uint32_t offA = (uint32_t)(mt * BM) * lda_b + lrow * lda_b + lchunk;
        const uint32_t offB = (uint32_t)(nt * BN - BM) * ldb_b + lrow * ldb_b + lchunk;
#pragma unroll
        for (int i = 0; i < DPW; ++i) {
            const uint32_t b = (uint32_t)(wave * DPW + i);
            const uint32_t dst = slot + b * 1024;
            const uint32_t voff = isA[i] ? offA + b * RPB * lda_b : offB + b * RPB * ldb_b;
            if (isA[i]) dma16(rA, dst, voff, soff);
            else dma16(rB, dst, voff, soff);
        }
    };

    // Fragment offsets inside a slot: row r = base + lane%16 (base a multiple
    // of 16), logical chunk lane/16 + 4·ks at physical chunk ^ (lane%8)
    // (128-byte rows) or ^ ((lane%16)/4) (64-byte rows).
    int fo[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
        fo[ks] = (lane & 15) * ROWB +
                 ((ROWB == 128 ? ((lane >> 4) + 4 * ks) ^ (lane & 7) : (lane >> 4) ^ ((lane >> 2) & 3)) << 4);
    const int abase = wm * MT * 16 * ROWB, bbase = BM * ROWB + wn * NTL * 16 * ROWB;

    using AccT = std::conditional_t<I8, i32x4, f32x4>;
    AccT acc[NTL][MT];
    auto clear = [&] {
#pragma unroll
        for (int a = 0; a < NTL; ++a)
#pragma unroll
            for (int b = 0; b < MT; ++b) acc[a][b] = AccT{};
    };
    clear();

    auto compute = [&](int slot) {
        const uint8_t *base = ring + slot * STAGE;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            i32x4 af[MT], bf[NTL];
#pragma unroll
            for (int t = 0; t < MT; ++t) af[t] = *(const i32x4 *)(base + abase + t * 16 * ROWB + fo[ks]);
#pragma unroll
            for (int t = 0; t < NTL; ++t) bf[t] = *(const i32x4 *)(base + bbase + t * 16 * ROWB + fo[ks]);
#pragma unroll
            for (int tn = 0; tn < NTL; ++tn)
#pragma unroll
                for (int tm = 0; tm < MT; ++tm) {
                    if constexpr (I8)
                        acc[tn][tm] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[tn], af[tm], acc[tn][tm], 0, 0, 0);
                    else
                        acc[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, bf[tn]),
                                                                             __builtin_bit_cast(f16x8, af[tm]),
                                                                             acc[tn][tm], 0, 0, 0);
                }
        }
    };

    // Epilogue of tile ti, in two parts.  epi_load issues the loads the
    // epilogue needs (column constants, binary16 residual rows, row statistics)
    // before the ring's DMA of the tile's last slice: a wait for a load queued
    // behind those DMAs would also wait for them.  epi_store does the
    // arithmetic, gemm.hip's epilogue_store term for term, and the stores:
    // buffer stores, whose range check drops rows past M, so every lane of
    // every wave issues exactly NSTORE of them.
    // This lane's 16 features: cb + 32·h + 4·half + {0..3}, q = 2·h + half.
    constexpr int ESZ = OUT_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t rC = buf_rsrc(g.C, (uint32_t)g.M * (uint32_t)g.ldc * ESZ);
    f32x4 k1[4], k2[4], kb[4], kg[4], kt[4], ksb[4];
    float ksa[MT];  // int8 scales: b_scale of this lane's columns, a_scale of its rows
    // With eight token tiles a wave the binary16 residual does not fit in
    // registers beside the last slice's operands: epi_store loads it instead
    // (its wait then also covers the next slice's DMA, issued before).
    constexpr bool LATE_RES = RES == 2 && MT > 4;
    f16x8 rh[MT][2];
    f32x2 sti[MT];  // (mean, rstd) of the row: A's (LN_IN) or the residual's (RES_LN)
    auto tile_of = [&](int ti, int &m0, int &nt) {
        const int t = t0 + ti * nbx;
        const int mt = t / cols;
        nt = col0 + t - mt * cols;
        m0 = mt * BM;
    };
    auto epi_load = [&](int ti) {
        int m0, nt;
        tile_of(ti, m0, nt);
        const int cb = nt * BN + wn * NTL * 16 + (lane >> 4) * 8;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int col = cb + (q >> 1) * 32 + (q & 1) * 4;
            if (LNM == fh::LN_IN) {
                k1[q] = *(const f32x4 *)(g.c1 + col);
                k2[q] = *(const f32x4 *)(g.c2 + col);
            }
            if (BIAS) kb[q] = *(const f32x4 *)(g.bias + col);
            if (I8) ksb[q] = *(const f32x4 *)(g.b_scale + col);
            if (LNM == fh::RES_LN) {
                kg[q] = *(const f32x4 *)(g.ln_g + col);
                kt[q] = *(const f32x4 *)(g.ln_b + col);
            }
        }
        // Rows past M are clamped to M−1: loaded, never stored.
#pragma unroll
        for (int tm = 0; tm < MT; ++tm) {
            const int rr = min(m0 + (wm * MT + tm) * 16 + (lane & 15), g.M - 1);
            if (RES == 2 && !LATE_RES) {
#pragma unroll
                for (int h = 0; h < 2; ++h) rh[tm][h] = *(const f16x8 *)(g.resid_h + (size_t)rr * g.ldr + cb + h * 32);
            }
            if (LNM != fh::LN_NONE) sti[tm] = g.stats_in[rr];
            if (I8) ksa[tm] = g.a_scale[rr];
        }
    };
    auto epi_store = [&](int ti) {
        int m0, nt;
        tile_of(ti, m0, nt);
        const int cb = nt * BN + wn * NTL * 16 + (lane >> 4) * 8;
        // An f32 residual (too many registers to hold across the last slice)
        // is loaded here, still ahead of the stores.
        // (late residual: two token tiles ahead of their use)
        auto load_rh = [&](int tm) {
            const int rr = min(m0 + (wm * MT + tm) * 16 + (lane & 15), g.M - 1);
#pragma unroll
            for (int h = 0; h < 2; ++h) rh[tm][h] = *(const f16x8 *)(g.resid_h + (size_t)rr * g.ldr + cb + h * 32);
        };
        if (LATE_RES) {
            load_rh(0);
            load_rh(1);
        }
        f32x4 rf[MT][4];
        if (RES == 1) {
#pragma unroll
            for (int tm = 0; tm < MT; ++tm) {
                const int rr = min(m0 + (wm * MT + tm) * 16 + (lane & 15), g.M - 1);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    rf[tm][q] = *(const f32x4 *)(g.resid + (size_t)rr * g.ldr + cb + (q >> 1) * 32 + (q & 1) * 4);
            }
        }
#pragma unroll
        for (int tm = 0; tm < MT; ++tm) {
            if (LATE_RES && tm + 2 < MT) load_rh(tm + 2);
            const uint32_t row = (uint32_t)(m0 + (wm * MT + tm) * 16 + (lane & 15));
            const f32x2 rs = LNM != fh::LN_NONE ? sti[tm] : (f32x2){0.f, 0.f};
            if constexpr (ACT == fh::ACT_SWIGLU) {
                // B holds up and gate rows interleaved in 16-row blocks, so
                // this lane's rows are the up (lanes < 32) or the gate
                // (lanes ≥ 32) rows of features f + 0..7 (q = 0, 1) and
                // f + 16 + 0..7 (q = 2, 3), f = 8·(lane/16 % 2), of the
                // 64-row block's 32 outputs, and lane l ^ 32 holds the other
                // rows of the same features.  After the fold and bias (each
                // lane its own columns' terms, as gemm.hip), a permlane32
                // swap leaves every lane both operands of one feature set:
                // lanes < 32 the first, lanes ≥ 32 the second.
                f32x4 xs[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    f32x4 x = acc[q][tm];
                    if (LNM == fh::LN_IN) x = ln_fold_v(x, rs, k1[q], k2[q]);
                    if (BIAS) x += kb[q];
                    xs[q] = x;
                }
                f16x8 o;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const f32x2 ug = swap_halves(xs[i >> 2][i & 3], xs[2 + (i >> 2)][i & 3]);
                    o[i] = to_f16(ug[0] * silu(ug[1]));
                }
                const int ocol = (cb & ~63) / 2 + (lane >> 5) * 16 + ((lane >> 4) & 1) * 8;
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, o), rC,
                                                       (row * (uint32_t)g.ldc + (uint32_t)ocol) * ESZ, 0, 0);
                continue;
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                f32x4 v[2];
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int q = 2 * h + half;
                    f32x4 x;
                    if constexpr (I8) {
                        // The scaled sum is rounded before the bias is added
                        // (gemm.hip's int8 epilogue; the empty asm keeps the
                        // compiler from fusing the two into one fma).
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            float v = __fmul_rn((float)acc[q][tm][i], __fmul_rn(ksa[tm], ksb[q][i]));
                            asm("" : "+v"(v));
                            x[i] = v;
                        }
                    } else {
                        x = acc[q][tm];
                    }
                    if (LNM == fh::LN_IN) x = ln_fold_v(x, rs, k1[q], k2[q]);
                    if (BIAS) x += kb[q];
                    if (ACT == fh::ACT_GELU) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) x[i] = gelu_erf(x[i]);
                    }
                    if (RES == 1) {
                        x += rf[tm][q];
                    } else if (RES == 2) {
                        const f16x8 r8 = rh[tm][h];
                        const f16x4 r4 = half ? (f16x4){r8[4], r8[5], r8[6], r8[7]} : (f16x4){r8[0], r8[1], r8[2], r8[3]};
                        if (LNM == fh::RES_LN) x += ln_resid_v(r4, rs, kg[q], kt[q]);
                        else x += (f32x4){(float)r4[0], (float)r4[1], (float)r4[2], (float)r4[3]};
                    }
                    v[half] = x;
                }
                const uint32_t off = (row * (uint32_t)g.ldc + (uint32_t)(cb + h * 32)) * ESZ;
                if (OUT_F32) {
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v[0]), rC, off, 0, 0);
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v[1]), rC, off + 16, 0, 0);
                } else {
                    f16x8 o;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        o[i] = to_f16(v[0][i]);
                        o[4 + i] = to_f16(v[1][i]);
                    }
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, o), rC, off, 0, 0);
                }
            }
        }
    };
    // Vector memory instructions epi_store issues after its loads.
    constexpr int NSTORE = ACT == fh::ACT_SWIGLU ? MT : MT * (OUT_F32 ? 4 : 2);

    // Ring: slice s lives in slot s % SLOTS; SLOTS−1 slices are in flight
    // while one is multiplied.  Before multiplying slice s this wave waits
    // until slice s's DMA has landed, then the barrier makes every wave's
    // part of slice s visible and frees the slot slice s−1 used, for slice
    // s+SLOTS−1.  Vector memory operations retire in order, so "slice s
    // landed" is "at most n younger operations outstanding".  Issued after
    // slice s's DMA (at iteration s−SLOTS+1): the DMA of slices s+1 ..
    // s+SLOTS−2, and the NSTORE stores of an epilogue that ended one of
    // slices s−SLOTS+1 .. s−1 (its loads have been consumed, so they are
    // not outstanding).  Counting more than were issued would not wait long
    // enough: n counts at most one epilogue.
    constexpr int NIN = (SLOTS - 2) * DPW;
#pragma unroll
    for (int i = 0; i < SLOTS - 1; ++i) issue();
    // kk: K position of slice s in its tile; since_end: slices since the
    // last tile end (an epilogue's stores are outstanding for the next
    // SLOTS − 1 slices).
    int kk = 0, ti = 0, slot = 0, since_end = SLOTS;
    for (int s = 0; s < nsl; ++s) {
        if (since_end < SLOTS) {
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NIN + NSTORE) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NIN) : "memory");
        }
        const bool tile_end = kk == nk - 1;
        if (tile_end) epi_load(ti);
        issue();
        compute(slot);
        slot = slot + 1 == SLOTS ? 0 : slot + 1;
        ++since_end;
        if (tile_end) {
            epi_store(ti);
            clear();
            kk = 0;
            ++ti;
            since_end = 1;
        } else {
            ++kk;
        }
    }
    // The DMA path writes this block's LDS: drain it before the block ends.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Column groups of the XCD tile split.  With 256-wide tiles and an even
// number of them, two groups: each XCD then streams half of B (at BERT-base's
// FFN1, 2.4 of 4.7 MB per XCD: fewer weight re-fetches into its 4 MB L2,
// ~1.5% faster); otherwise one.  FUTON_RING_CG=1, 2 or 4 overrides (tuning
// knob; ignored where it does not divide the column tiles).
int ring_col_groups(int ntn, int bn) {
    static const int v = [] {
        const char *e = getenv("FUTON_RING_CG");
        return e ? atoi(e) : 0;
    }();
    const int c = v == 1 || v == 2 || v == 4 ? v : bn == 256 ? 2 : 1;
    return ntn % c == 0 ? c : 1;
}

template <class R, int ACT, bool OUT_F32, int LNM, bool BIAS, int RES, bool I8 = false>
hipError_t launch_ring(const GemmArgs &g, hipStream_t s) {
    const int ncu = fh::cu_count();
    if (ncu <= 0) return hipErrorUnknown;
    if (g.N % R::BN) return hipErrorInvalidValue;
    const int ntn = g.N / R::BN;
    const long ntiles = (long)((g.M + R::BM - 1) / R::BM) * ntn;
    // A multiple of 8 blocks (whole XCD groups); persistent: as many as the
    // CUs hold at once.
    const long all = (ntiles + 7) / 8 * 8;
    const int grid = (int)(R::PERSIST ? std::min<long>((long)(ncu / 8) * 8 * R::BPC, all) : all);
    const int cg = ring_col_groups(ntn, R::BN);
    const int per_part = (int)((ntiles / cg + 8 / cg - 1) / (8 / cg));
    hipLaunchKernelGGL((ring_kernel<R, ACT, OUT_F32, LNM, BIAS, RES, I8>), dim3(grid), dim3(R::NT), 0, s, g, ntn, per_part,
                       cg);
    return hipGetLastError();
}

// Selects the kernel for g's bias and residual pointers.
template <class R, int ACT, bool OUT_F32, int LNM>
hipError_t launch_ring_r(const GemmArgs &g, hipStream_t s) {
    const int res = g.resid ? 1 : g.resid_h ? 2 : 0;
    if (ACT == fh::ACT_RES16 || LNM == fh::RES_LN) {  // binary16 residual by construction
        return g.bias ? launch_ring<R, ACT, OUT_F32, LNM, true, 2>(g, s) : launch_ring<R, ACT, OUT_F32, LNM, false, 2>(g, s);
    }
    if (LNM == fh::LN_IN || res == 0) {
        return g.bias ? launch_ring<R, ACT, OUT_F32, LNM, true, 0>(g, s) : launch_ring<R, ACT, OUT_F32, LNM, false, 0>(g, s);
    }
    if (res == 1) {
        return g.bias ? launch_ring<R, ACT, OUT_F32, LNM, true, 1>(g, s) : launch_ring<R, ACT, OUT_F32, LNM, false, 1>(g, s);
    }
    return hipErrorInvalidValue;  // a binary16 residual outside ACT_RES16
}

// Configurations (measured on the 18k-token bge-small projections, op level:
// R0 30.2 µs for QKV, R1 27.8, R2 25.0, R3 32.9, R4 32.7).  R2 runs two
// persistent 4-wave blocks per CU: while one block waits at its barrier or
// runs its epilogue, the other keeps the matrix cores busy.  R5's 256×256
// tiles need half the operand bytes per MFMA of R2's 128×128 (the slices
// stream from L2 at ~16 B/clk per CU on the 65k-token BERT-base projections:
// R5 is 12–14% faster there).  R6 measured slower than R5 (same stream rate,
// twice the barriers).
using R0 = RCfg<256, 128, 4, 2, 3, true>;   // 8 waves, 3 slots, one persistent block per CU
using R1 = RCfg<128, 128, 2, 2, 2, false>;  // 4 waves, 2 slots, one block per tile (two per CU)
using R2 = RCfg<128, 128, 2, 2, 2, true>;   // R1's blocks, persistent, two per CU
using R3 = RCfg<128, 128, 4, 2, 3, true>;   // 8 waves of 32×64, 3 slots, persistent
using R4 = RCfg<256, 128, 4, 2, 3, false>;  // R0's tile, one block per tile
using R5 = RCfg<256, 256, 2, 4, 2, true>;   // 8 waves of 128×64, 2 slots, one persistent block per CU
using R6 = RCfg<256, 256, 2, 4, 5, true, 64>;  // R5's tile, 5 slots of 32-wide K slices

// FUTON_RING_CFG=0..6 forces a configuration (tuning knob); unset: R5 where
// its tiles fit (N a multiple of 256, no f32 residual) and cover at least
// three quarters of the CUs (nomic-bert's 240-tile output projections: 6–11%
// faster than R2's 960 smaller tiles), else R2.
int ring_cfg() {
    static const int v = [] {
        const char *e = getenv("FUTON_RING_CFG");
        const int c = e ? atoi(e) : -1;
        return c >= 0 && c <= 6 ? c : -1;
    }();
    return v;
}

template <int ACT, bool OUT_F32, int LNM>
hipError_t launch_ring(const GemmArgs &g, hipStream_t s) {
    const bool fit256 = g.N % R5::BN == 0 && !g.resid;
    switch (ring_cfg()) {
    case 0: return launch_ring_r<R0, ACT, OUT_F32, LNM>(g, s);
    case 1: return launch_ring_r<R1, ACT, OUT_F32, LNM>(g, s);
    case 2: return launch_ring_r<R2, ACT, OUT_F32, LNM>(g, s);
    case 3: return launch_ring_r<R3, ACT, OUT_F32, LNM>(g, s);
    case 4: return launch_ring_r<R4, ACT, OUT_F32, LNM>(g, s);
    case 5: return fit256 ? launch_ring_r<R5, ACT, OUT_F32, LNM>(g, s) : launch_ring_r<R2, ACT, OUT_F32, LNM>(g, s);
    case 6:
        return fit256 && LNM != fh::RES_LN ? launch_ring_r<R6, ACT, OUT_F32, LNM>(g, s)
                                           : launch_ring_r<R2, ACT, OUT_F32, LNM>(g, s);
    default:
        if (fit256 && 4L * ((g.M + R5::BM - 1) / R5::BM) * (g.N / R5::BN) >= 3L * fh::cu_count())
            return launch_ring_r<R5, ACT, OUT_F32, LNM>(g, s);
        return launch_ring_r<R2, ACT, OUT_F32, LNM>(g, s);
    }
}

// The int8 forms (no LayerNorm fold): f32 residual (f32 output) or none.
template <class R, int ACT, bool OUT_F32>
hipError_t launch_ring_q8_r(const GemmArgs &g, hipStream_t s) {
    if constexpr (R::BN == 256 || !OUT_F32) {  // no f32 residual here (launch_ring_q8, gemm_ring_q8_ok)
        if (g.resid) return hipErrorInvalidValue;
    } else if (g.resid) {
        return g.bias ? launch_ring<R, ACT, true, fh::LN_NONE, true, 1, true>(g, s)
                      : launch_ring<R, ACT, true, fh::LN_NONE, false, 1, true>(g, s);
    }
    return g.bias ? launch_ring<R, ACT, OUT_F32, fh::LN_NONE, true, 0, true>(g, s)
                  : launch_ring<R, ACT, OUT_F32, fh::LN_NONE, false, 0, true>(g, s);
}

template <int ACT, bool OUT_F32>
hipError_t launch_ring_q8(const GemmArgs &g, hipStream_t s) {
    const bool fit256 = g.N % R5::BN == 0 && !g.resid;
    const int c = ring_cfg();
    if (c == 5 && fit256) return launch_ring_q8_r<R5, ACT, OUT_F32>(g, s);
    if (c < 0 && fit256 && 4L * ((g.M + R5::BM - 1) / R5::BM) * (g.N / R5::BN) >= 3L * fh::cu_count())
        return launch_ring_q8_r<R5, ACT, OUT_F32>(g, s);
    return launch_ring_q8_r<R2, ACT, OUT_F32>(g, s);
}

// out row r ← B row ring_pack_row(r), 16 bytes per thread.
__global__ void ring_pack_kernel(const f16 *__restrict__ B, f16 *__restrict__ out, int N, int K) {
    const long c = (long)blockIdx.x * blockDim.x + threadIdx.x, cpr = K / 8;
    if (c >= (long)N * cpr) return;
    const int r = (int)(c / cpr), ch = (int)(c - (long)r * cpr);
    *(f16x8 *)(out + (size_t)r * K + ch * 8) = *(const f16x8 *)(B + (size_t)fh::ring_pack_row(r) * K + ch * 8);
}

}  // namespace

namespace fh {

hipError_t ring_pack(const f16 *B, f16 *out, int N, int K, hipStream_t s) {
    if (N % 64 || K % 8 || N <= 0 || K <= 0) return hipErrorInvalidValue;
    const long n = (long)N * (K / 8);
    hipLaunchKernelGGL(ring_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, B, out, N, K);
    return hipGetLastError();
}

bool gemm_ring_worth(int M, int N) {
    // Enough 128×128 tiles for about half of the two-per-CU block slots.
    return N % BN == 0 && (long)((M + 127) / 128) * (N / BN) >= 192;
}

bool gemm_ring_ok(const GemmArgs &g, int act, bool out_f32, int ln) {
    if (g.M <= 0 || g.N % BN != 0 || g.K % 64 != 0 || g.K <= 0 || g.res_map) return false;
    if (act != ACT_NONE && act != ACT_GELU && act != ACT_RES16 && act != ACT_SWIGLU) return false;
    // SwiGLU: binary16 out, ldc ≥ N/2, no residual
    if (act == ACT_SWIGLU && (out_f32 || g.resid || g.resid_h || ln == RES_LN || g.ldc < g.N / 2)) return false;
    if (g.lda % 8 || g.ldb % 8 || g.ldc % 8 || ((g.resid || g.resid_h) && g.ldr % 8)) return false;
    if (act == ACT_RES16 && (out_f32 || !g.resid_h)) return false;
    if (ln == LN_IN && (out_f32 || g.resid || g.resid_h)) return false;
    if (act != ACT_RES16 && ln != RES_LN && g.resid_h && !g.resid) return false;
    if (ln == RES_LN && (out_f32 || !g.resid_h || g.resid)) return false;
    // 32-bit buffer offsets: every row the ring addresses (up to M + BM − 1).
    if (((double)g.M + BM_MAX) * g.lda * 2.0 >= 2147483648.0 || (double)g.N * g.ldb * 2.0 >= 2147483648.0) return false;
    if (((double)g.M + BM_MAX) * g.ldc * (out_f32 ? 4.0 : 2.0) >= 2147483648.0) return false;
    return true;
}

bool gemm_ring_q8_ok(const GemmArgs &g, int act, bool out_f32) {
    if (g.res_map) return false;
    if (g.M <= 0 || g.N % BN != 0 || g.K % 128 != 0 || g.K <= 0) return false;
    if (act != ACT_NONE && act != ACT_GELU) return false;
    if (!g.a_scale || !g.b_scale || g.resid_h || (g.resid && !out_f32)) return false;
    if (g.lda % 16 || g.ldb % 16 || g.ldc % 8 || (g.resid && g.ldr % 4)) return false;
    // 32-bit buffer offsets: every row the ring addresses (up to M + BM − 1).
    if (((double)g.M + BM_MAX) * g.lda >= 2147483648.0 || (double)g.N * g.ldb >= 2147483648.0) return false;
    if (((double)g.M + BM_MAX) * g.ldc * (out_f32 ? 4.0 : 2.0) >= 2147483648.0) return false;
    return true;
}

hipError_t gemm_ring_q8(const GemmArgs &a, int act, bool out_f32, hipStream_t s) {
    if (!gemm_ring_q8_ok(a, act, out_f32)) return hipErrorInvalidValue;
    if (out_f32) return act == ACT_GELU ? launch_ring_q8<ACT_GELU, true>(a, s) : launch_ring_q8<ACT_NONE, true>(a, s);
    return act == ACT_GELU ? launch_ring_q8<ACT_GELU, false>(a, s) : launch_ring_q8<ACT_NONE, false>(a, s);
}

hipError_t gemm_ring(const GemmArgs &a, int act, bool out_f32, hipStream_t s, int ln) {
    if (act == ACT_NONE && !out_f32 && a.resid_h && !a.resid) act = ACT_RES16;
    if (!gemm_ring_ok(a, act, out_f32, ln)) return hipErrorInvalidValue;
    if (ln == LN_IN) {
        if (act == ACT_NONE) return launch_ring<ACT_NONE, false, LN_IN>(a, s);
        if (act == ACT_GELU) return launch_ring<ACT_GELU, false, LN_IN>(a, s);
        if (act == ACT_SWIGLU) return launch_ring<ACT_SWIGLU, false, LN_IN>(a, s);
        return hipErrorInvalidValue;
    }
    if (ln == RES_LN) return launch_ring<ACT_RES16, false, RES_LN>(a, s);
    if (act == ACT_RES16) return launch_ring<ACT_RES16, false, LN_NONE>(a, s);
    if (act == ACT_SWIGLU) return launch_ring<ACT_SWIGLU, false, LN_NONE>(a, s);
    if (act == ACT_GELU)
        return out_f32 ? launch_ring<ACT_GELU, true, LN_NONE>(a, s) : launch_ring<ACT_GELU, false, LN_NONE>(a, s);
    return out_f32 ? launch_ring<ACT_NONE, true, LN_NONE>(a, s) : launch_ring<ACT_NONE, false, LN_NONE>(a, s);
}

}  // namespace fh
