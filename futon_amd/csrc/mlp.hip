// Fused feed-forward block of the encoder layer on gfx950 (hidden width 384):
//   h   = GELU(LN(y)·W1ᵀ + b1)          (native/model.go:607-620)
//   out = h·W2ᵀ + b2 + LN(y)           (native/model.go:622-633)
// with LN(y) folded as in the separate GEMMs (W1 stored scaled by γ, the fold
// terms c1/c2, y's row statistics from row_stats).  h never leaves the CU: it
// is produced 128 intermediate features at a time into LDS and consumed there
// by the second product, which saves the [M, I] binary16 round trip through
// HBM and one launch per layer.
//
// Layout and schedule, one 8-wave block per BM = 16·MT tokens:
// * The block's token tile y[BM, 384] is DMA'd into LDS once (buffer_load …
//   lds) and stays resident; rows past M read as zero.  LDS rows are 128
//   bytes with the 16-byte chunk index XOR-ed with row%8, so MFMA fragment
//   reads (16 rows × one chunk) are conflict-free.
// * Weights never pass through LDS: both matrices are stored as 1-KB MFMA
//   operand fragments in the order each wave consumes them (mlp_w1_unit,
//   mlp_w2_unit), and every wave loads its own fragments straight into
//   registers ahead of use (W1 half a chunk, W2 a chunk).  Each weight byte
//   is read once per block.
// * v_mfma_f32_16x16x32_f16, weights as the A operand.  Per 128-feature chunk
//   j, wave w: phase 1 computes features 16w .. 16w+15 for all BM tokens;
//   its epilogue (LayerNorm fold, GELU, rounding to binary16) writes h into
//   LDS; after one barrier, phase 2 accumulates outputs 48w .. 48w+47 over
//   the chunk's 128 features.  h is double-buffered, so that barrier is the
//   chunk's only one, and each chunk's epilogue (the VALU-heavy part) runs
//   interleaved with the previous chunk's phase 2.  The fold terms c1/c2 are
//   staged in LDS once per block.
// * On gfx950 a wave64 VALU instruction issued beside the MFMA stream hides
//   under it only about once per MFMA, so this kernel's time is close to its
//   MFMA time plus its vector time; what pays is fewer vector instructions
//   and no exposed memory latency, not where the vector work is placed.
// The accumulation orders over K and the epilogue arithmetic are those of the
// ring GEMM's LN_IN/GELU and RES_LN forms, so the result has the same bits as
// the two separate GEMMs.
#include <algorithm>
#include <type_traits>

#include "fh_common.h"
#include "gemm_epi.h"
#include "lds_dma.h"
#include "row_stats.h"

namespace {
using namespace fh_epi;
using fh_dma::buf_rsrc;
using fh_dma::dma16;

constexpr int HD = 384;                 // hidden width
constexpr int KB1 = HD / 64;            // 64-wide k-blocks of the token tile
constexpr int CH = 128;                 // intermediate features per chunk
constexpr int KS1 = HD / 32;            // phase-1 k-steps per chunk
constexpr int KS2 = CH / 32;            // phase-2 k-steps per chunk
constexpr int W1H = KS1 / 2;            // W1 k-steps held in registers
constexpr int NW = fh::MLP_NW;              // waves per block
constexpr int NT1 = fh::MLP_NT1;            // phase-1 feature tiles per wave
constexpr int NT2 = fh::MLP_NT2;            // phase-2 output tiles per wave
constexpr int ROWB = 128;               // bytes per LDS row (64 binary16)
constexpr int MT_MAX = 5;
constexpr int PW = 6;                   // Wo k-steps held in registers (phase 0)
constexpr int QD = 4;                   // Wq k-steps held in registers (QKV passes)
constexpr int I_MAX = 2048;             // widest intermediate layer (fold terms staged in LDS)
constexpr int W1C = NW * KS1 * NT1 * 64;  // 16-byte units of W1 per chunk
constexpr int W2C = NW * KS2 * NT2 * 64;  // 16-byte units of W2 per chunk
static_assert(CH == NW * 16 * NT1 && NT2 * 16 * NW == HD, "wave split");

// MODE 0: the block from y; 1: with the output projection ahead of it
// (OUTP); 2: also with the next layer's QKV projection after it (QKVN).
template <int MT, bool BIAS, int MODE>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) void mlp_kernel(MlpArgs g) {
    constexpr bool OUTP = MODE >= 1, QKVN = MODE == 2;
    constexpr int BM = 16 * MT;
    constexpr int A_BYTES = KB1 * BM * ROWB;        // token tile, k-block major
    constexpr int H_BYTES = (CH / 64) * BM * ROWB;  // one chunk's h, k-block major
    // LDS: the token tile; region R, holding the attention tile (phase 0),
    // then the two h buffers (the chunk loop), then the output tile (same
    // layout as the token tile); the fold terms c1/c2, staged at entry; the
    // row statistics.
    constexpr int O_OFF = A_BYTES, R_BYTES = 2 * H_BYTES > A_BYTES ? 2 * H_BYTES : A_BYTES;
    constexpr int C_OFF = A_BYTES + R_BYTES;        // c1 [I_MAX] then c2 [I_MAX] (f32)
    constexpr int S_OFF = C_OFF + 2 * I_MAX * 4;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S_OFF + BM * 8];
    const uint8_t *const atile = lds;
    const float *const lc1 = (const float *)(lds + C_OFF), *const lc2 = lc1 + I_MAX;
    f32x2 *const lst = (f32x2 *)(lds + S_OFF);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m0 = blockIdx.x * BM;
    const int nchunk = g.I / CH;

    // This wave's weight fragments of chunk j: W1 (ks, tn), W2 (ks, t).  W1
    // is held half a chunk ahead: slot ks % W1H holds k-step ks, refilled with
    // k-step ks + W1H (of the same chunk, or ks − W1H of the next) once
    // consumed.  W2 is held a whole chunk ahead.
    const i32x4 *w1p = (const i32x4 *)g.w1 + (size_t)wave * KS1 * NT1 * 64 + lane;
    const i32x4 *w2p = (const i32x4 *)g.w2 + (size_t)wave * KS2 * NT2 * 64 + lane;
    i32x4 w1f[W1H][NT1], w2f[KS2][NT2];
    auto prefetch_w = [&] {
#pragma unroll
        for (int ks = 0; ks < W1H; ++ks)
#pragma unroll
            for (int tn = 0; tn < NT1; ++tn) w1f[ks][tn] = w1p[(ks * NT1 + tn) * 64];
#pragma unroll
        for (int ks = 0; ks < KS2; ++ks)
#pragma unroll
            for (int t = 0; t < NT2; ++t) w2f[ks][t] = w2p[(ks * NT2 + t) * 64];
    };
    // After multiplying k-step ks of chunk c: refill its slot.
    auto w1_refill = [&](int c, int ks) {
        const int cc = ks < W1H ? c : min(c + 1, nchunk - 1), kk = ks < W1H ? ks + W1H : ks - W1H;
#pragma unroll
        for (int tn = 0; tn < NT1; ++tn) w1f[ks % W1H][tn] = w1p[(size_t)cc * W1C + (kk * NT1 + tn) * 64];
    };
    // Row statistics of the tile's rows, when given (rows past M clamped:
    // never stored).
    if (!OUTP && g.stats && (int)threadIdx.x < BM) lst[threadIdx.x] = g.stats[min(m0 + (int)threadIdx.x, g.M - 1)];

    // DMA of a [BM, 384] binary16 tile of rows m0.. into LDS at `dst`
    // (k-block major, the swizzled layout): block b = rows 8·(b % 2MT) .. of
    // k-block b / 2MT, lane l writing physical chunk l%8 of row l/8, i.e.
    // logical chunk (l%8) ^ (l/8); blocks wave, wave + NW, ...  Rows past M
    // read as zero.  Then the fold terms c1, c2 (1 KB per block, lane-linear).
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)lds;
    auto dma_tile = [&](const f16 *src, uint32_t dst) {
        const __amdgpu_buffer_rsrc_t rs = buf_rsrc(src, (uint32_t)g.M * (HD * 2));
        const uint32_t lrow = lane >> 3, lchunk = ((lane & 7) ^ (lane >> 3)) * 16;
#pragma unroll
        for (int i = 0; i < (12 * MT + NW - 1) / NW; ++i) {
            const int b = wave + NW * i, kb = b / (2 * MT), rb = b - kb * 2 * MT;
            if (b < 12 * MT)
                dma16(rs, dst + (uint32_t)b * 1024, (uint32_t)(m0 + rb * 8 + (int)lrow) * (HD * 2) + lchunk,
                      (uint32_t)kb * ROWB);
        }
    };
    auto dma_fold_terms = [&] {
        const __amdgpu_buffer_rsrc_t rC1 = buf_rsrc(g.c1, (uint32_t)g.I * 4);
        const __amdgpu_buffer_rsrc_t rC2 = buf_rsrc(g.c2, (uint32_t)g.I * 4);
        const int ncb = (g.I * 4 + 1023) / 1024;
        for (int b = wave; b < 2 * ncb; b += NW) {
            const int which = b >= ncb, kb = b - which * ncb;
            dma16(which ? rC2 : rC1, lds0 + C_OFF + (uint32_t)which * (I_MAX * 4) + (uint32_t)kb * 1024,
                  (uint32_t)lane * 16, (uint32_t)kb * 1024);
        }
    };
    // Fragment offsets inside a 16-row group: row lane%16, logical chunk
    // lane/16 + 4·(ks%2) at physical chunk ^ (lane%8).
    int fo[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) fo[k] = (lane & 15) * ROWB + ((((lane >> 4) + 4 * k) ^ (lane & 7)) << 4);
    // MFMA B fragments of k-step k of a resident [BM, 384] tile: one b128
    // per 16-token group.
    auto load_tile_frags = [&](i32x4(&f)[MT], const uint8_t *tile, int k) {
        const uint8_t *ab = tile + (k >> 1) * BM * ROWB + fo[k & 1];
#pragma unroll
        for (int t = 0; t < MT; ++t) f[t] = *(const i32x4 *)(ab + t * 16 * ROWB);
    };

    if constexpr (OUTP) {
        // Phase 0, the attention output projection (the out-projection GEMM's
        // RES_LN form, same K order and epilogue arithmetic): the attention
        // tile goes to region R, Wo fragments stream through registers PW
        // k-steps ahead, and yB = attn·Woᵀ + bo + LN_a(ya) is written in
        // binary16 into the token tile, over ya, which was transferred
        // there.  This lane's outputs: the same n0 + {0..4·NT2−1} as the
        // final epilogue.
        // Issue order: the attention tile, the first PW k-steps of Wo, then
        // ya, the fold terms, bo/γ/β and ya's statistics.  vmcnt retires in
        // issue order, so waiting until no more than the Wo loads and the
        // smallest per-wave count of ya transfers remain outstanding means
        // this wave's attention transfers have landed; the rest lands under
        // the products (the compiler waits for register loads before their
        // use; the empty asm statements keep the groups in this order).
        dma_tile(g.attn, lds0 + O_OFF);
        asm volatile("" ::: "memory");
        const i32x4 *w0p = (const i32x4 *)g.wo + (size_t)wave * KS2 * NT2 * 64 + lane;
        i32x4 w0f[PW][NT2];
        auto wo_frag = [&](int k, int t) { return w0p[(size_t)(k / KS2) * W2C + ((k % KS2) * NT2 + t) * 64]; };
#pragma unroll
        for (int ks = 0; ks < PW; ++ks)
#pragma unroll
            for (int t = 0; t < NT2; ++t) w0f[ks][t] = wo_frag(ks, t);
        asm volatile("" ::: "memory");
        dma_tile(g.ya, lds0);
        dma_fold_terms();
        const int n0 = wave * 16 * NT2 + (lane >> 4) * 4 * NT2;
        f32x4 kb[NT2], kg[NT2], kt[NT2];
        f32x2 sa[MT];
#pragma unroll
        for (int t = 0; t < NT2; ++t) {
            if (g.bo) kb[t] = *(const f32x4 *)(g.bo + n0 + 4 * t);
            kg[t] = *(const f32x4 *)(g.ga + n0 + 4 * t);
            kt[t] = *(const f32x4 *)(g.ba + n0 + 4 * t);
        }
#pragma unroll
        for (int tm = 0; tm < MT; ++tm) sa[tm] = g.stats_a[min(m0 + tm * 16 + (lane & 15), g.M - 1)];
        constexpr int AFTER = NT2 * PW + 12 * MT / NW;  // issued after the last attention transfer, at least
        static_assert(AFTER <= 63, "vmcnt immediate");
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(AFTER) : "memory");
        f32x4 acc0[NT2][MT];
        i32x4 af0[2][MT];
        load_tile_frags(af0[0], lds + O_OFF, 0);
#pragma unroll
        for (int k = 0; k < KS1; ++k) {
            if (k + 1 < KS1) load_tile_frags(af0[(k + 1) & 1], lds + O_OFF, k + 1);
            __builtin_amdgcn_sched_barrier(0);
            const i32x4(&af)[MT] = af0[k & 1];
#pragma unroll
            for (int t = 0; t < NT2; ++t) {
#pragma unroll
                for (int tm = 0; tm < MT; ++tm)
                    acc0[t][tm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(f16x8, w0f[k % PW][t]), __builtin_bit_cast(f16x8, af[tm]),
                        k == 0 ? (f32x4){0.f, 0.f, 0.f, 0.f} : acc0[t][tm], 0, 0, 0);
                if (k + PW < KS1) w0f[k % PW][t] = wo_frag(k + PW, t);
            }
        }
        // The block's weights are requested now, to land under the epilogue
        // and the statistics; ya's transfers are waited for (every wave's).
        asm volatile("" ::: "memory");
        prefetch_w();
        constexpr int NPF = W1H * NT1 + KS2 * NT2;  // the loads of prefetch_w
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(NPF) : "memory");
#pragma unroll
        for (int tm = 0; tm < MT; ++tm) {
            const int r = tm * 16 + (lane & 15);
#pragma unroll
            for (int t = 0; t < NT2; ++t) {
                const int n = n0 + 4 * t;
                f32x4 x = acc0[t][tm];
                if (g.bo) x += kb[t];
                f16x4 *const p = (f16x4 *)(lds + (n >> 6) * BM * ROWB + r * ROWB + ((((n & 63) >> 3) ^ (lane & 7)) << 4) +
                                           (n & 7) * 2);
                x += ln_resid_v(*p, sa[tm], kg[t], kt[t]);
                f16x4 o;
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] = to_f16(x[i]);
                *p = o;
            }
        }
        // yB is complete.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
        prefetch_w();
        dma_tile(g.y, lds0);
        dma_fold_terms();
        // Everything above has landed (the weights were requested first, so
        // their latency overlaps the tile's) and every wave's part is visible.
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    // (mean, rstd) of a tile's rows in row_stats' order: 16 lanes per row,
    // lane l16 holding 16-byte chunks c·16 + l16; each row's result goes to
    // dst(r, stats) from lane 0 of each row.  The conditions are uniform per
    // wave (BM % 4 == 0).
    auto tile_stats = [&](const uint8_t *tile, int lane, auto dst) {
        const int l16 = lane & 15;
#pragma unroll
        for (int r0 = 0; r0 < BM; r0 += NW * 4) {
            const int r = r0 + wave * 4 + (lane >> 4);
            if (r0 + wave * 4 < BM) {
                f16x8 v[HD / 128];
#pragma unroll
                for (int c = 0; c < HD / 128; ++c) {
                    const int q = c * 16 + l16;
                    v[c] = *(const f16x8 *)(tile + (q >> 3) * BM * ROWB + r * ROWB + (((q & 7) ^ (r & 7)) << 4));
                }
                const f32x2 st = fh_rs::row_stats16<HD / 128>(v, g.eps);
                if (l16 == 0) dst(r, st);
            }
        }
    };
    if (OUTP || !g.stats) {
        tile_stats(atile, lane, [&](int r, f32x2 st) { lst[r] = st; });
        // (with OUTP also the fold terms and weights requested above)
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    // Chunk-local phase-1 features of this lane: fl .. fl + 4·NT1 − 1.
    const int fl = wave * 16 * NT1 + (lane >> 4) * 4 * NT1;

    f32x4 acc1[NT1][MT], acc2[NT2][MT];  // phase-1 product of one chunk, the block's output
#pragma unroll
    for (int tm = 0; tm < MT; ++tm)
#pragma unroll
        for (int t = 0; t < NT2; ++t) acc2[t][tm] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // Token fragments of phase-1 k-step ks, and h fragments of phase-2
    // k-step ks from h buffer hb: one b128 per 16-token tile.
    auto load_af = [&](i32x4(&f)[MT], int ks) {
        const uint8_t *ab = atile + (ks >> 1) * BM * ROWB + fo[ks & 1];
#pragma unroll
        for (int t = 0; t < MT; ++t) f[t] = *(const i32x4 *)(ab + t * 16 * ROWB);
    };
    auto load_hf = [&](i32x4(&f)[MT], const uint8_t *hb, int ks) {
        const uint8_t *hr = hb + (ks >> 1) * BM * ROWB + fo[ks & 1];
#pragma unroll
        for (int t = 0; t < MT; ++t) f[t] = *(const i32x4 *)(hr + t * 16 * ROWB);
    };
    // Phase-1 epilogue of token tile tm of chunk c (acc holds its finished
    // product): fold, GELU, binary16, into h buffer c % 2 at this lane's
    // 4·NT1 features.
    auto epi1_tm = [&](int tm, const f32x4(&acc)[NT1][MT], int c) {
        const f32x2 sv = lst[tm * 16 + (lane & 15)];
        _Float16 o[4 * NT1] __attribute__((aligned(16)));
#pragma unroll
        for (int tn = 0; tn < NT1; ++tn) {
            const f32x4 k1 = *(const f32x4 *)(lc1 + c * CH + fl + 4 * tn);
            const f32x4 k2 = *(const f32x4 *)(lc2 + c * CH + fl + 4 * tn);
            const f32x4 x = ln_fold_v(acc[tn][tm], sv, k1, k2);
#pragma unroll
            for (int i = 0; i < 4; ++i) o[4 * tn + i] = to_f16(gelu_erf(x[i]));
        }
        const int row = tm * 16 + (lane & 15);
        uint8_t *dst = lds + A_BYTES + (c & 1) * H_BYTES + (fl >> 6) * BM * ROWB + row * ROWB +
                       ((((fl & 63) >> 3) ^ (lane & 7)) << 4) + (fl & 7) * 2;
        if (NT1 == 2) *(f16x8 *)dst = *(const f16x8 *)o;
        else *(f16x4 *)dst = *(const f16x4 *)o;
    };

    // Phase 1 of chunk c into acc (W1 fragments · token tileᵀ), refilling W1
    // with the fragments half a chunk ahead.  The token fragments of k-step
    // ks + 1 are requested before the products of k-step ks (register double
    // buffer; the scheduling barrier keeps that order): this stage has no
    // other work to cover the LDS latency.
    auto p1_chunk = [&](int c, f32x4(&acc)[NT1][MT]) {
        i32x4 af[2][MT];
        load_af(af[0], 0);
#pragma unroll
        for (int ks = 0; ks < KS1; ++ks) {
            if (ks + 1 < KS1) load_af(af[(ks + 1) & 1], ks + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int tn = 0; tn < NT1; ++tn)
#pragma unroll
                for (int tm = 0; tm < MT; ++tm)
                    acc[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(f16x8, w1f[ks % W1H][tn]), __builtin_bit_cast(f16x8, af[ks & 1][tm]),
                        ks == 0 ? (f32x4){0.f, 0.f, 0.f, 0.f} : acc[tn][tm], 0, 0, 0);
            w1_refill(c, ks);
        }
    };

    // Chunk 0's phase 1 and its epilogue; its W1 registers are refilled with
    // chunk 1's fragments.
    p1_chunk(0, acc1);
#pragma unroll
    for (int tm = 0; tm < MT; ++tm) epi1_tm(tm, acc1, 0);

    // Chunk j: stage A multiplies chunk j+1's phase 1 into accN (refilling W1
    // with chunk j+2's fragments); one barrier (chunk j's h is complete);
    // stage B multiplies chunk j's phase 2 (refilling W2 with chunk j+1's)
    // beside chunk j+1's epilogue, interleaved with the products (one MFMA,
    // then a share of the epilogue).  h is double-buffered: chunk j+1's h goes
    // to the buffer chunk j−1 used, read by every wave before it passed this
    // chunk's barrier.  MORE (compile time, so neither stage branches): chunk
    // j+1 exists.  (Moving part of the epilogue into stage A measured no
    // faster: MFMA and VALU issue share the SIMD, so where the vector work
    // sits matters less than how much of it there is.)
    auto chunk = [&](int j, f32x4(&accN)[NT1][MT], auto more_c) {
        constexpr bool MORE = decltype(more_c)::value;
        if constexpr (MORE) p1_chunk(j + 1, accN);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const uint8_t *hb = lds + A_BYTES + (j & 1) * H_BYTES;
        const size_t next2 = (size_t)min(j + 1, nchunk - 1) * W2C;
#pragma unroll
        for (int ks = 0; ks < KS2; ++ks) {
            i32x4 hf[MT];
            load_hf(hf, hb, ks);
#pragma unroll
            for (int t = 0; t < NT2; ++t) {
#pragma unroll
                for (int tm = 0; tm < MT; ++tm)
                    acc2[t][tm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(f16x8, w2f[ks][t]), __builtin_bit_cast(f16x8, hf[tm]), acc2[t][tm], 0, 0, 0);
                w2f[ks][t] = w2p[next2 + (ks * NT2 + t) * 64];
            }
            if constexpr (MORE) {
#pragma unroll
                for (int tm = ks * MT / KS2; tm < (ks + 1) * MT / KS2; ++tm) epi1_tm(tm, accN, j + 1);
                // One epilogue tile is ~80 VALU instructions: spread them
                // between the k-step's NT2·MT products (groups of one MFMA and
                // a share of the VALU work; the counts must be constants).
                const int ntile = (ks + 1) * MT / KS2 - ks * MT / KS2;
                if (ntile == 1) {
#pragma unroll
                    for (int i = 0; i < NT2 * MT; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
                    }
                } else if (ntile == 2) {
#pragma unroll
                    for (int i = 0; i < NT2 * MT; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 11, 0);
                    }
                }
            }
        }
    };
    int j = 0;
    for (; j + 1 < nchunk; ++j) chunk(j, acc1, std::true_type{});
    chunk(j, acc1, std::false_type{});

    // The next layer's Wq fragments (k-step kg of the 3·KS1-step stream over
    // the three 384-row blocks, tile t), the first QD requested now so their
    // latency overlaps the output stage; its fold terms c1q/c2q go to the
    // fold-term region (free: every wave has passed the chunk loop's last
    // barrier, so no epilogue reads c1/c2 any more).
    const i32x4 *wqp = (const i32x4 *)g.wq + (size_t)wave * KS2 * NT2 * 64 + lane;
    auto wq_frag = [&](int kg, int t) {
        const int p = kg / KS1, k = kg - p * KS1;
        return wqp[(size_t)p * (HD * HD / 8) + (size_t)(k / KS2) * W2C + ((k % KS2) * NT2 + t) * 64];
    };
    i32x4 wqf[QD][NT2];
    if constexpr (QKVN) {
        const __amdgpu_buffer_rsrc_t rQ1 = buf_rsrc(g.c1q, 3 * HD * 4), rQ2 = buf_rsrc(g.c2q, 3 * HD * 4);
        constexpr int NCB = (3 * HD * 4 + 1023) / 1024;
        for (int b = wave; b < 2 * NCB; b += NW) {
            const int which = b >= NCB, kb = b - which * NCB;
            dma16(which ? rQ2 : rQ1, lds0 + C_OFF + (uint32_t)which * (I_MAX * 4) + (uint32_t)kb * 1024,
                  (uint32_t)lane * 16, (uint32_t)kb * 1024);
        }
#pragma unroll
        for (int ks = 0; ks < QD; ++ks)
#pragma unroll
            for (int t = 0; t < NT2; ++t) wqf[ks][t] = wq_frag(ks, t);
    }

    {
    // The lane id again, opaque to the compiler: the output stage recomputes
    // its LDS offsets instead of keeping the prologue's identical ones alive
    // (in spill slots) across the chunk loop.
    int lane = threadIdx.x & 63;
    asm volatile("" : "+v"(lane));
    // Output epilogue: acc + b2 + (y − mean)·rstd·γ + β, rounded once; y read
    // back from the resident token tile.  This lane's outputs:
    // n0 = 16·NT2·wave + 4·NT2·(lane/16) + {0 .. 4·NT2 − 1}.  The binary16
    // results go to the output tile in LDS (the h/c region, free once every
    // wave has left the chunk loop), whose rows are then stored with 16-byte
    // coalesced stores and, when asked, reduced to their statistics.
    const int n0 = wave * 16 * NT2 + (lane >> 4) * 4 * NT2;
    f32x4 kb[NT2], kg[NT2], kt[NT2];
#pragma unroll
    for (int t = 0; t < NT2; ++t) {
        if (BIAS) kb[t] = *(const f32x4 *)(g.b2 + n0 + 4 * t);
        kg[t] = *(const f32x4 *)(g.ln_g + n0 + 4 * t);
        kt[t] = *(const f32x4 *)(g.ln_b + n0 + 4 * t);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    uint8_t *const otile = lds + O_OFF;
#pragma unroll
    for (int tm = 0; tm < MT; ++tm) {
        const int r = tm * 16 + (lane & 15);
        const f32x2 sv = lst[r];
#pragma unroll
        for (int t = 0; t < NT2; ++t) {
            const int n = n0 + 4 * t;
            const int off = (n >> 6) * BM * ROWB + r * ROWB + ((((n & 63) >> 3) ^ (lane & 7)) << 4) + (n & 7) * 2;
            const f16x4 y4 = *(const f16x4 *)(atile + off);
            f32x4 x = acc2[t][tm];
            if (BIAS) x += kb[t];
            x += ln_resid_v(y4, sv, kg[t], kt[t]);
            f16x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = to_f16(x[i]);
            *(f16x4 *)(otile + off) = o;
        }
    }
    // (with QKVN also the fold-term transfers)
    if constexpr (QKVN) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // Rows [BM, 384] of an LDS tile in the swizzled layout to rows of `rs`
    // (row pitch `pitch` bytes, column offset `col` bytes), 16-byte coalesced
    // stores; rows past M are dropped by the buffer bounds.
    auto store_tile = [&](const uint8_t *tile, __amdgpu_buffer_rsrc_t rs, int pitch, int col) {
        constexpr int UPR = HD * 2 / 16;  // 16-byte units per row
        for (int u = (int)threadIdx.x; u < BM * UPR; u += 64 * NW) {
            const int r = u / UPR, cu = u - r * UPR;
            const i32x4 v = *(const i32x4 *)(tile + (cu >> 3) * BM * ROWB + r * ROWB + (((cu & 7) ^ (r & 7)) << 4));
            __builtin_amdgcn_raw_buffer_store_b128(v, rs, (uint32_t)((m0 + r) * pitch + col + cu * 16), 0, 0);
        }
    };
    store_tile(otile, buf_rsrc(g.out, (uint32_t)g.M * (HD * 2)), HD * 2, 0);
    auto out_stats = [&] {
        tile_stats(otile, lane, [&](int r, f32x2 st) {
            if (g.stats_out && m0 + r < g.M) g.stats_out[m0 + r] = st;
            if (QKVN) lst[r] = st;  // every wave has read y's statistics (barrier above)
        });
    };
    if constexpr (!QKVN) {
        if (g.stats_out) out_stats();
    } else {
        // The next layer's QKV projection of the output tile (the QKV GEMM's
        // LN_IN form: same K order, same fold arithmetic), 384 columns per
        // pass.  The three passes are one stream of 3·KS1 k-steps for the Wq
        // ring (QD k-steps ahead), so a pass's epilogue overlaps the next
        // pass's loads.  The output tile's statistics, which only the
        // epilogues need, are computed beside the first pass's products.  A
        // pass's binary16 results are staged in the token tile (free after
        // the output epilogue) and stored as whole rows.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const __amdgpu_buffer_rsrc_t rQ = buf_rsrc(g.qkv, (uint32_t)g.M * (3 * HD * 2));
        uint8_t *const stile = lds;
#pragma unroll
        for (int p = 0; p < 3; ++p) {
            f32x4 accq[NT2][MT];
            i32x4 afq[2][MT];
            load_tile_frags(afq[0], otile, 0);
#pragma unroll
            for (int k = 0; k < KS1; ++k) {
                const int kg = p * KS1 + k;  // position in the stream
                if (k + 1 < KS1) load_tile_frags(afq[(k + 1) & 1], otile, k + 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = 0; t < NT2; ++t) {
#pragma unroll
                    for (int tm = 0; tm < MT; ++tm)
                        accq[t][tm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(f16x8, wqf[kg % QD][t]), __builtin_bit_cast(f16x8, afq[k & 1][tm]),
                            k == 0 ? (f32x4){0.f, 0.f, 0.f, 0.f} : accq[t][tm], 0, 0, 0);
                    if (kg + QD < 3 * KS1) wqf[kg % QD][t] = wq_frag(kg + QD, t);
                }
                if (p == 0 && k == 1) out_stats();
            }
            // The statistics (pass 0) are visible, and every wave has read
            // the previous pass's staged rows.
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            f32x4 kc1[NT2], kc2[NT2];
#pragma unroll
            for (int t = 0; t < NT2; ++t) {
                kc1[t] = *(const f32x4 *)(lc1 + p * HD + n0 + 4 * t);
                kc2[t] = *(const f32x4 *)(lc2 + p * HD + n0 + 4 * t);
            }
#pragma unroll
            for (int tm = 0; tm < MT; ++tm) {
                const int r = tm * 16 + (lane & 15);
                const f32x2 sv = lst[r];
#pragma unroll
                for (int t = 0; t < NT2; ++t) {
                    const f32x4 x = ln_fold_v(accq[t][tm], sv, kc1[t], kc2[t]);
                    f16x4 o;
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[i] = to_f16(x[i]);
                    const int n = n0 + 4 * t;
                    *(f16x4 *)(stile + (n >> 6) * BM * ROWB + r * ROWB + ((((n & 63) >> 3) ^ (lane & 7)) << 4) +
                               (n & 7) * 2) = o;
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            store_tile(stile, rQ, 3 * HD * 2, p * HD * 2);
        }
    }
    }
}

// out = the fragment-ordered copy of B, 16 bytes per thread.
__global__ void mlp_pack_kernel(int kind, const f16 *__restrict__ B, f16 *__restrict__ out, int N, int K) {
    const long u = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= (long)N * K / 8) return;
    int row, col;
    if (kind == 1) fh::mlp_w1_unit(u, K, row, col);
    else fh::mlp_w2_unit(u, K, row, col);
    *(f16x8 *)(out + u * 8) = *(const f16x8 *)(B + (size_t)row * K + col);
}

template <int MT>
hipError_t launch_mlp(const MlpArgs &g, hipStream_t s) {
    const int grid = (g.M + 16 * MT - 1) / (16 * MT);
    const int mode = g.attn ? (g.wq ? 2 : 1) : 0;
    switch (mode * 2 + (g.b2 ? 1 : 0)) {
    case 0: hipLaunchKernelGGL((mlp_kernel<MT, false, 0>), dim3(grid), dim3(64 * NW), 0, s, g); break;
    case 1: hipLaunchKernelGGL((mlp_kernel<MT, true, 0>), dim3(grid), dim3(64 * NW), 0, s, g); break;
    case 2: hipLaunchKernelGGL((mlp_kernel<MT, false, 1>), dim3(grid), dim3(64 * NW), 0, s, g); break;
    case 3: hipLaunchKernelGGL((mlp_kernel<MT, true, 1>), dim3(grid), dim3(64 * NW), 0, s, g); break;
    case 4: hipLaunchKernelGGL((mlp_kernel<MT, false, 2>), dim3(grid), dim3(64 * NW), 0, s, g); break;
    default: hipLaunchKernelGGL((mlp_kernel<MT, true, 2>), dim3(grid), dim3(64 * NW), 0, s, g); break;
    }
    return hipGetLastError();
}

}  // namespace

namespace fh {

int cu_count() {
    static int ncu = 0;
    if (ncu == 0) {
        int dev = 0;
        hipDeviceProp_t p;
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) return 0;
        ncu = p.multiProcessorCount;
    }
    return ncu;
}

hipError_t mlp_pack(int kind, const f16 *B, f16 *out, int N, int K, hipStream_t s) {
    if (N <= 0 || K <= 0 || !(kind == 1 ? N % (16 * NT1) == 0 && K % 32 == 0 : kind == 2 && N % HD == 0 && K % CH == 0))
        return hipErrorInvalidValue;
    const long n = (long)N * (K / 8);
    hipLaunchKernelGGL(mlp_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, kind, B, out, N, K);
    return hipGetLastError();
}

bool mlp_ok(int M, int H, int I) {
    // 32-bit buffer offsets for y/out (M·768 bytes) and the weights.
    return H == HD && I > 0 && I % CH == 0 && I <= I_MAX && M > 0 && (double)M * HD * 2 < 2147483648.0 &&
           (double)I * HD * 2 < 2147483648.0;
}

bool mlp_qkv_ok(int M) { return M > 0 && (double)M * 3 * HD * 2 < 2147483648.0; }

hipError_t mlp(const MlpArgs &g, hipStream_t s) {
    if (!mlp_ok(g.M, HD, g.I) || !g.w1 || !g.c1 || !g.c2 || !g.w2 || !g.ln_g || !g.ln_b || !g.out)
        return hipErrorInvalidValue;
    if (g.attn ? !g.wo || !g.ya || !g.stats_a || !g.ga || !g.ba || g.stats : !g.y) return hipErrorInvalidValue;
    if (g.wq && (!g.attn || !g.c1q || !g.c2q || !g.qkv || !mlp_qkv_ok(g.M))) return hipErrorInvalidValue;
    const int ncu = fh::cu_count();
    if (ncu <= 0) return hipErrorUnknown;
    // Tokens per block: the fewest 16-row tiles that cover M with one block
    // per CU (weights are re-read once per block, so fewer, larger blocks).
    const int mt = std::min(MT_MAX, std::max(1, (g.M + 16 * ncu - 1) / (16 * ncu)));
    switch (mt) {
    case 1: return launch_mlp<1>(g, s);
    case 2: return launch_mlp<2>(g, s);
    case 3: return launch_mlp<3>(g, s);
    case 4: return launch_mlp<4>(g, s);
    default: return launch_mlp<5>(g, s);
    }
}

}  // namespace fh
