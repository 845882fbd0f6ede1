// Varlen multi-head self-attention over packed sequences on gfx950 MFMA.
//
// Replaces the reference's per-head attendHead + softmaxScaled
// (native/model.go:646-739): scores = q·kᵀ, softmax(scores/√d) per query
// row, out = P·v, written to the head's columns of the concatenated output.
// The reference runs each sequence unpadded; here sequences are packed
// back to back (offsets[]) and every key outside the query's own sequence
// is excluded, which is the same function.  RoPE (rotateHalf,
// model.go:705-712) is applied to q (in registers) and k (in LDS).
//
// Block = (query group, head, sequence); each wave owns QT tiles of 16
// queries.  K and V of a KBLK-key block are staged once per block in LDS
// (V transposed).  Each wave computes Sᵀ = K·Qᵀ with
// v_mfma_f32_16x16x32_f16 so that a lane owns four scores of ONE query
// (lane%16): the online-softmax statistics of a query live in the lanes
// that also own its output column, and P feeds the Oᵀ = Vᵀ·Pᵀ MFMA straight
// from registers (the key order inside the contraction is permuted
// identically on both operands).  Q fragments are loaded from global memory
// directly in the MFMA operand layout.
#include <cstdlib>
#include <type_traits>

#include "fh_common.h"

namespace {

#ifndef ATTN_PAIR_ORDER
#define ATTN_PAIR_ORDER 1
#endif
#ifndef ATTN_ONE_WAVES
#define ATTN_ONE_WAVES 6
#endif
// Long-kernel block shapes (waves × query tiles per wave) at head width 64:
// 8 × 2 while the longest sequence has at most ATTN_LONG_SPLIT tokens, 4 × 3
// beyond; 4 × 2 at head width 32.
#ifndef ATTN_LONG_SPLIT
#define ATTN_LONG_SPLIT 1024
#endif

// Sequences past one key block take the pipelined kernel (attn_long_kernel)
// unless FUTON_ATTN_LONG=0 (read per launch; diagnostics and the
// bit-equality test against attn_kernel's multi-block path).
bool long_pipeline() {
    const char *e = getenv("FUTON_ATTN_LONG");
    return !(e && e[0] == '0');
}

// With one key block and 32-wide heads the kernel fits in 80 VGPRs without
// spills: ask for six waves per SIMD (four at the compiler's own choice of
// 107 VGPRs), so more of the many short (sequence, head) blocks are resident.
// Blocks of fewer than four waves are held to fewer per SIMD by their LDS.
template <int D, int WAVES, bool ONE>
constexpr int attn_min_waves() { return (ONE && D == 32 && WAVES >= 4) ? ATTN_ONE_WAVES : 1; }

// Cross-row reductions of a lane's value with lane l^16 / l^32 through
// gfx950's row-swap permutes (no LDS crossbar, unlike ds_bpermute): with
// both operands x, permlane16_swap returns {x[l], x[l^16]} in every lane and
// permlane32_swap {x[l], x[l^32]}, so max and sum of the pair are what
// __shfl_xor would give, bit for bit (both operations are commutative).
// Operands and results pass through empty asm statements: this compiler
// otherwise folds a float max or sum of the two results as if both were the
// first (it drops the operation).
template <int ROWS>
__device__ __forceinline__ f32x2 swap_pair(float v) {
    unsigned a = __builtin_bit_cast(unsigned, v), b = a;
    asm volatile("" : "+v"(b));
    const auto r = ROWS == 16 ? __builtin_amdgcn_permlane16_swap(a, b, false, false)
                              : __builtin_amdgcn_permlane32_swap(a, b, false, false);
    unsigned r0 = r[0], r1 = r[1];
    asm volatile("" : "+v"(r0), "+v"(r1));
    return (f32x2){__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1)};
}
__device__ __forceinline__ float max_xor16(float v) {
    const f32x2 p = swap_pair<16>(v);
    return fmaxf(p[0], p[1]);
}
__device__ __forceinline__ float max_xor32(float v) {
    const f32x2 p = swap_pair<32>(v);
    return fmaxf(p[0], p[1]);
}
__device__ __forceinline__ float sum_xor16(float v) {
    const f32x2 p = swap_pair<16>(v);
    return p[0] + p[1];
}
__device__ __forceinline__ float sum_xor32(float v) {
    const f32x2 p = swap_pair<32>(v);
    return p[0] + p[1];
}

// Per query (lane%16), the sum of a key block's binary16 probabilities held
// as the MFMA B operand (pf[c]: 32 keys per chunk): ones·Pᵀ on the matrix
// cores, each row of the result tile the column sum.  Used where the block's
// probabilities are summed for the softmax denominator (the kernels with
// several key blocks); it normalizes by exactly the weights PV multiplies.
template <int NC>
__device__ __forceinline__ float prob_sum(const f16x8 (&pf)[NC]) {
    const f16x8 ones = {(f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f, (f16)1.f};
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pf[c], acc, 0, 0, 0);
    return acc[0];
}

// Block ids reach the 8 XCDs round-robin; remap them so each XCD gets a
// contiguous range of (query group, head, sequence) items, ordered so that
// blocks which read the same qkv lines share one L2 (the lines are then
// fetched once, not once per XCD).
__device__ __forceinline__ void block_item(const AttnArgs &a, int &seq, int &head, int &qg) {
    const int gx = gridDim.x, gy = gridDim.y, nb = gx * gy * gridDim.z;
    const int pid = (blockIdx.z * gy + blockIdx.y) * gx + blockIdx.x;
    const int xcd = pid & 7, idx = pid >> 3, q8 = nb >> 3, r8 = nb & 7;
    const int logical = xcd * q8 + min(xcd, r8) + idx;
    qg = logical % gx;
    const int t = logical / gx;
    if (ATTN_PAIR_ORDER && (gy & 1) == 0) {
        // (head pair, sequence, head) order: the two heads whose q/k/v
        // segments share 128-byte lines stay on one XCD, and each XCD's
        // range spans many sequences, so per-XCD work varies less than with
        // whole sequences per XCD.
        const int nseq = gridDim.z, u = t >> 1;
        head = (u / nseq) * 2 + (t & 1);
        seq = u % nseq;
    } else {
        head = t % gy;
        seq = t / gy;
    }
    seq += a.seq0;
}

// The long kernel's mapping at head widths of 64 and more (a head's q/k/v
// segment is then a whole 128-byte line, so head pairs share nothing):
// units u = (sequence, head) are dealt round-robin to the XCDs (unit u on XCD
// u mod 8) and every query group of a unit runs on the unit's XCD, where its
// K/V rows are fetched into one L2.  Each XCD thus gets interleaved heads of
// every sequence and the same share of work whatever the sequence lengths
// (contiguous ranges of sequences differ by up to 13% per XCD at 512..2048
// tokens).  The 1-D grid holds gx·8·ceil(units/8) blocks; false: no unit.
__device__ __forceinline__ bool block_unit(const AttnArgs &a, int gx, int units, int &seq, int &head, int &qg) {
    const int pid = blockIdx.x, xcd = pid & 7, idx = pid >> 3;
    const int u = xcd + 8 * (idx / gx);
    qg = idx - (idx / gx) * gx;
    if (u >= units) return false;
    const int heads = a.H / a.d;
    seq = u / heads + a.seq0;
    head = u - (u / heads) * heads;
    return true;
}

// rotateHalf's two products and their difference (first half) or sum
// (second half), each rounded to float32 on its own as the reference's Go
// code computes them, the same in every kernel: contraction into a fused
// multiply-add is switched off here (hipcc contracts by default, and the
// __f*_rn helpers are plain operators in this toolchain).
__device__ __forceinline__ float rot(float x, float partner, float cs, float sn, bool first) {
#pragma clang fp contract(off)
    const float a = x * cs, b = partner * sn;
    return first ? a - b : a + b;
}

// rotateHalf applied in place to the binary16 Q and K of every token
// (model.go:705-712): the same rot and rounding the attention kernels apply
// while loading Q and staging K, so attention run afterwards without RoPE
// gives the same bits, and K is rotated once per token instead of once per
// query block that stages it.  Thread u of sequence blockIdx.y handles token
// u / UPT of the sequence and one 8-wide chunk c of dims (c·8 .. +8, and the
// partners half away) of one head of Q or of K; half % 8 == 0.
__global__ __launch_bounds__(256) void rope_qk_kernel(f16 *__restrict__ qkv, const int32_t *__restrict__ offsets,
                                                       int H, int d, const float *__restrict__ cos_t,
                                                       const float *__restrict__ sin_t) {
    const int seq = blockIdx.y, start = offsets[seq], L = offsets[seq + 1] - start;
    const int half = d >> 1, cph = half / 8, heads = H / d, upt = 2 * heads * cph;
    const long u = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= (long)L * upt) return;
    const int p = (int)(u / upt), r = (int)(u - (long)p * upt);
    const int region = r / (heads * cph), hc = r - region * heads * cph, head = hc / cph, c = hc - head * cph;
    f16 *x = qkv + (size_t)(start + p) * 3 * H + region * H + head * d + c * 8;
    const f16x8 a = *(const f16x8 *)x, b = *(const f16x8 *)(x + half);
    const float *cp = cos_t + (size_t)p * half + c * 8, *sp = sin_t + (size_t)p * half + c * 8;
    f16x8 lo, hi;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float x1 = (float)a[e], x2 = (float)b[e], cs = cp[e], sn = sp[e];
        lo[e] = (f16)rot(x1, x2, cs, sn, true);
        hi[e] = (f16)rot(x2, x1, cs, sn, false);
    }
    *(f16x8 *)x = lo;
    *(f16x8 *)(x + half) = hi;
}

// Q fragments of QT 16-query tiles (B operand of Sᵀ = K·Qᵀ): lane holds
// dims [dk·32 + (lane/16)·8, +8) of query lane%16 of each tile, rotated
// (rotateHalf, model.go:705-712) when the pack uses RoPE.
template <int D, int QT, bool ROPE>
__device__ __forceinline__ void load_q(const AttnArgs &a, int start, int L, int qbase, int lane,
                                       f16x8 (&qf)[QT][D / 32], int head) {
    const int d = a.d, half = d >> 1, ld = 3 * a.H;
    const f16x8 z8 = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int q = min(qbase + qt * 16 + (lane & 15), L - 1);
        const f16 *qrow = a.qkv + (size_t)(start + q) * ld + head * d;
#pragma unroll
        for (int dk = 0; dk < D / 32; ++dk) {
            const int j0 = dk * 32 + (lane >> 4) * 8;
            f16x8 v = z8;
            if (j0 < d) v = *(const f16x8 *)(qrow + j0);
            if (ROPE && j0 < d) {
                // Partner dims j ± half: inside this chunk when half < 8 (d = 8),
                // else the aligned chunk half away.
                f16x8 p = v;
                if (half >= 8) p = *(const f16x8 *)(qrow + (j0 < half ? j0 + half : j0 - half));
                f16x8 r;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int j = j0 + e;
                    const int i = j < half ? j : j - half;  // table index
                    const float cs = a.rope_cos[q * half + i], sn = a.rope_sin[q * half + i];
                    float partner;
                    if (half >= 8) partner = (float)p[e];
                    else partner = (float)v[(e + half) & 7];
                    const float x = (float)v[e];
                    r[e] = (f16)rot(x, partner, cs, sn, j < half);
                }
                v = r;
            }
            qf[qt][dk] = v;
        }
    }
}

template <int D, int WAVES, int QT, int KBLK, bool OUT_F32, bool ROPE, bool ONE>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(attn_min_waves<D, WAVES, ONE>(), 8)))
void attn_kernel(AttnArgs a) {
    // ONE: every sequence fits in one key block (L <= KBLK), so each query
    // tile is finished (softmax, PV, normalise, store) before the next one
    // starts and only one tile's output and statistics are live at a time.
    // The arithmetic is the same as the multi-block path's first block
    // (running max -inf, running sum 0), so the results are the same bits.
    constexpr int QROWS = 16 * QT * WAVES;
    constexpr int QS = ONE ? 1 : QT;  // query tiles with live softmax state
    constexpr int KS = D + 8;     // K LDS row stride (halves)
    constexpr int VS = KBLK + 8;  // Vᵀ LDS row stride (halves)
    constexpr int NKT = KBLK / 16;
    static_assert(KBLK % 32 == 0, "PV consumes 32-key chunks");
    __shared__ __attribute__((aligned(16))) f16 Ks[KBLK * KS];
    __shared__ __attribute__((aligned(16))) f16 Vt[D * VS];

    int seq, head, qg;
    block_item(a, seq, head, qg);
    const int start = a.offsets[seq];
    const int L = a.offsets[seq + 1] - start;
    const int nq = min(L, a.q_limit);
    const int q0 = qg * QROWS;
    if (q0 >= nq) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int d = a.d, H = a.H, ld = 3 * H;
    const int half = d >> 1;
    const int chunks = d >> 3;  // 16-byte chunks per row (d % 8 == 0)
    const f16x8 z8 = {0, 0, 0, 0, 0, 0, 0, 0};

    // ── Q fragments (B operand of Sᵀ = K·Qᵀ): lane holds dims
    //    [dk·32 + (lane/16)·8, +8) of query lane%16 of each tile (load_q's
    //    arithmetic, written out here: this kernel's register allocation
    //    spills with the shared helper). ──
    f16x8 qf[QT][D / 32];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int q = min(q0 + (wave * QT + qt) * 16 + (lane & 15), L - 1);
        const f16 *qrow = a.qkv + (size_t)(start + q) * ld + head * d;
#pragma unroll
        for (int dk = 0; dk < D / 32; ++dk) {
            const int j0 = dk * 32 + (lane >> 4) * 8;
            f16x8 v = z8;
            if (j0 < d) v = *(const f16x8 *)(qrow + j0);
            if (ROPE && j0 < d) {
                f16x8 p = v;
                if (half >= 8) p = *(const f16x8 *)(qrow + (j0 < half ? j0 + half : j0 - half));
                f16x8 r;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int j = j0 + e;
                    const int i = j < half ? j : j - half;  // table index
                    const float cs = a.rope_cos[q * half + i], sn = a.rope_sin[q * half + i];
                    float partner;
                    if (half >= 8) partner = (float)p[e];
                    else partner = (float)v[(e + half) & 7];
                    r[e] = (f16)rot((float)v[e], partner, cs, sn, j < half);
                }
                v = r;
            }
            qf[qt][dk] = v;
        }
    }

    f32x4 o[QS][D / 16];
    float m_run[QS], l_run[QS];
    auto reset = [&](int st) {
        m_run[st] = -INFINITY;
        l_run[st] = 0.f;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) o[st][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    };
#pragma unroll
    for (int st = 0; st < QS; ++st) reset(st);
    const float sl2 = a.scale_log2e;

    // Lane owns O[query lane%16][dims t·16 + (lane/16)·4 .. +4] of each tile.
    auto store = [&](int qt, int st) {
        const int q = q0 + (wave * QT + qt) * 16 + (lane & 15);
        if (q >= nq) return;
        const float inv = 1.0f / l_run[st];
        const size_t orow = a.compact ? (size_t)seq : (size_t)(start + q);
#pragma unroll
        for (int t = 0; t < D / 16; ++t) {
            const int dim = t * 16 + (lane >> 4) * 4;
            if (dim >= d) continue;
            const f32x4 v = o[st][t] * inv;
            if (OUT_F32) {
                *(f32x4 *)((float *)a.out + orow * a.ldo + head * d + dim) = v;
            } else {
                const f16x4 h = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
                *(f16x4 *)((f16 *)a.out + orow * a.ldo + head * d + dim) = h;
            }
        }
    };

    for (int kb0 = 0; kb0 < L; kb0 += KBLK) {
        if (kb0 > 0) __syncthreads();  // previous block's K/V fully consumed
        // Stage only the key rows the MFMAs read: whole 32-key PV chunks
        // that hold a valid key (rows past L repeat the last key: finite).
        const int rows = min(KBLK, (L - kb0 + 31) & ~31);
        // One key block: each thread owns a fixed set of (key pair, chunk)
        // items, so all of its K/V loads are issued before the first LDS
        // store (row indices clamped to the last key instead of branching),
        // and Vᵀ is written as packed key pairs (32-bit stores).
        constexpr int CPR = D / 8;               // 16-byte chunks per row
        constexpr int PAIRS = KBLK / 2 * CPR;    // (key pair, chunk) items
        constexpr int NP = PAIRS / (WAVES * 64);
        constexpr bool PAIRED = ONE && PAIRS % (WAVES * 64) == 0 && NP <= 4;
        if constexpr (PAIRED) {
            f16x8 k0[NP], k1[NP], v0[NP], v1[NP];
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int c = i * WAVES * 64 + tid, p = c / CPR;
                const int chl = min(c % CPR, chunks - 1);
                const f16 *r0 = a.qkv + (size_t)(start + min(2 * p, L - 1)) * ld + head * d + chl * 8;
                const f16 *r1 = a.qkv + (size_t)(start + min(2 * p + 1, L - 1)) * ld + head * d + chl * 8;
                k0[i] = *(const f16x8 *)(r0 + H);
                k1[i] = *(const f16x8 *)(r1 + H);
                v0[i] = *(const f16x8 *)(r0 + 2 * H);
                v1[i] = *(const f16x8 *)(r1 + 2 * H);
            }
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                const int c = i * WAVES * 64 + tid, p = c / CPR, ch = c % CPR;
                if (2 * p >= rows) continue;  // rows is a multiple of 32: pairs never straddle it
                const bool live = ch < chunks;
                const f16x8 ka = live ? k0[i] : z8, kb = live ? k1[i] : z8;
                const f16x8 va = live ? v0[i] : z8, vb = live ? v1[i] : z8;
                *(f16x8 *)&Ks[(2 * p) * KS + ch * 8] = ka;
                *(f16x8 *)&Ks[(2 * p + 1) * KS + ch * 8] = kb;
#pragma unroll
                for (int j = 0; j < 8; ++j) *(f16x2 *)&Vt[(ch * 8 + j) * VS + 2 * p] = (f16x2){va[j], vb[j]};
            }
        } else
        for (int c = tid; c < rows * (D / 8); c += WAVES * 64) {
            const int r = c / (D / 8), ch = c % (D / 8);
            const int key = min(kb0 + r, L - 1);
            const f16 *row = a.qkv + (size_t)(start + key) * ld + head * d + ch * 8;
            f16x8 kv = z8, vv = z8;
            if (ch < chunks) {
                kv = *(const f16x8 *)(row + H);
                vv = *(const f16x8 *)(row + 2 * H);
            }
            *(f16x8 *)&Ks[r * KS + ch * 8] = kv;
#pragma unroll
            for (int j = 0; j < 8; ++j) Vt[(ch * 8 + j) * VS + r] = vv[j];
        }
        __syncthreads();
        if (ROPE) {
            for (int c = tid; c < rows * half; c += WAVES * 64) {
                const int r = c / half, i = c % half;
                const int pos = min(kb0 + r, L - 1);
                const float cs = a.rope_cos[pos * half + i], sn = a.rope_sin[pos * half + i];
                const float x1 = (float)Ks[r * KS + i], x2 = (float)Ks[r * KS + i + half];
                Ks[r * KS + i] = (f16)rot(x1, x2, cs, sn, true);
                Ks[r * KS + i + half] = (f16)rot(x2, x1, cs, sn, false);
            }
            __syncthreads();
        }
        const int kvalid = L - kb0;                   // valid keys from kb0 on
        const int nkt = min(NKT, (kvalid + 15) >> 4);  // key tiles holding valid keys

        // One query tile against this key block's NV valid key tiles (NV is
        // uniform across the block, so each count gets its own straight-line
        // code: scores, exponentials and PV chunks only for valid keys, the
        // mask only on the last tile).
        auto qtile = [&](auto nv_c, int qt) {
            constexpr int NV = decltype(nv_c)::value;
            const int st = ONE ? 0 : qt;
            constexpr int NC = (NV + 1) / 2;  // 32-key PV chunks
            // Sᵀ tiles: s[kt][i] = score(key kb0 + kt·16 + (lane/16)·4 + i, query lane%16).
            f32x4 s[NV];
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < NV; ++kt) {
                s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int dk = 0; dk < D / 32; ++dk) {
                    const f16x8 kf = *(const f16x8 *)&Ks[(kt * 16 + (lane & 15)) * KS + dk * 32 + (lane >> 4) * 8];
                    s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[qt][dk], s[kt], 0, 0, 0);
                }
                if (kt == NV - 1 && kt * 16 + 16 > kvalid) {  // boundary tile: mask keys past the sequence
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (kt * 16 + (lane >> 4) * 4 + i >= kvalid) s[kt][i] = -INFINITY;
                }
                mx = fmaxf(mx, fmaxf(fmaxf(s[kt][0], s[kt][1]), fmaxf(s[kt][2], s[kt][3])));
            }
            mx = max_xor32(max_xor16(mx));
            const float m_new = fmaxf(m_run[st], mx * sl2);  // log2-scaled running max
            const float corr = __builtin_amdgcn_exp2f(m_run[st] - m_new);
            float psum = 0.f;
            f16x8 pf[NC];
#pragma unroll
            for (int kt = 0; kt < 2 * NC; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = kt < NV ? __builtin_amdgcn_exp2f(s[kt < NV ? kt : 0][i] * sl2 - m_new) : 0.f;
                    if (ONE) psum += p;
                    pf[kt >> 1][(kt & 1) * 4 + i] = (f16)p;
                }
            // Several key blocks: the block's probability sum per query on
            // the matrix cores, from the binary16 probabilities PV uses
            // (ones·Pᵀ, every row of the tile the sum), as attn_long_kernel.
            if (ONE) psum = sum_xor32(sum_xor16(psum));
            else psum = prob_sum<NC>(pf);
            l_run[st] = l_run[st] * corr + psum;
            m_run[st] = m_new;
#pragma unroll
            for (int t = 0; t < D / 16; ++t) o[st][t] *= corr;

            // Oᵀ += Vᵀ·Pᵀ over 32-key chunks; key slots {4g..4g+3, 16+4g..16+4g+3}, g = lane/16.
#pragma unroll
            for (int c = 0; c < NC; ++c) {
#pragma unroll
                for (int t = 0; t < D / 16; ++t) {
                    const f16 *vrow = &Vt[(t * 16 + (lane & 15)) * VS + c * 32 + (lane >> 4) * 4];
                    const f16x4 lo = *(const f16x4 *)vrow;
                    const f16x4 hi = *(const f16x4 *)(vrow + 16);
                    const f16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    o[st][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[c], o[st][t], 0, 0, 0);
                }
            }
        };
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            if (q0 + (wave * QT + qt) * 16 >= nq) continue;  // tile holds no live query (wave-uniform)
            if (ONE) reset(0);
            static_assert(NKT <= 8, "key tiles per block");
            switch (nkt) {
            case 1: qtile(std::integral_constant<int, 1>{}, qt); break;
            case 2: qtile(std::integral_constant<int, 2>{}, qt); break;
            case 3: if constexpr (NKT >= 3) qtile(std::integral_constant<int, (NKT >= 3 ? 3 : 1)>{}, qt); break;
            case 4: if constexpr (NKT >= 4) qtile(std::integral_constant<int, (NKT >= 4 ? 4 : 1)>{}, qt); break;
            case 5: if constexpr (NKT >= 5) qtile(std::integral_constant<int, (NKT >= 5 ? 5 : 1)>{}, qt); break;
            case 6: if constexpr (NKT >= 6) qtile(std::integral_constant<int, (NKT >= 6 ? 6 : 1)>{}, qt); break;
            case 7: if constexpr (NKT >= 7) qtile(std::integral_constant<int, (NKT >= 7 ? 7 : 1)>{}, qt); break;
            default: qtile(std::integral_constant<int, NKT>{}, qt); break;
            }
            if (ONE) store(qt, 0);
        }
    }
    if (!ONE) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) store(qt, qt);
    }
}

// Sequences longer than one key block, head width exactly D: the same
// per-query arithmetic as attn_kernel's multi-block path (Sᵀ = K·Qᵀ per
// 16-key tile, one online-softmax update per 64-key block, Oᵀ += Vᵀ·Pᵀ over
// 32-key chunks, keys past the sequence masked to −∞), so both give the same
// bits, with the key blocks pipelined: the next block's K and V are fetched
// into registers while the current one is multiplied, rotated (RoPE) and
// transposed in registers, and written to the other half of a
// double-buffered LDS stage — one barrier per key block.  Each wave owns QT
// query tiles, so a block stages each key block once for 16·QT·WAVES
// queries.
template <int D, int WAVES, int QT, bool OUT_F32, bool ROPE>
__global__ __launch_bounds__(WAVES * 64) void attn_long_kernel(AttnArgs a, int gx, int units) {
    constexpr int BK = 64, NKT = BK / 16, NC = BK / 32;
    constexpr int NT = WAVES * 64, QROWS = 16 * QT * WAVES;
    constexpr int KS = D + 8, VS = BK + 8;  // LDS row pitches (halves)
    constexpr int CPR = D / 8, HCH = CPR / 2;  // 16-byte chunks per row; RoPE partner distance in chunks
    // K items: (key, chunk), or with RoPE (key, chunk pair c / c + HCH);
    // V items: (key pair, chunk), written as Vᵀ key pairs.
    constexpr int KI = ROPE ? BK * HCH : BK * CPR, VI = BK / 2 * CPR;
    constexpr int NKI = (KI + NT - 1) / NT, NVI = (VI + NT - 1) / NT;
    __shared__ __attribute__((aligned(16))) f16 Ks[2][BK * KS];
    __shared__ __attribute__((aligned(16))) f16 Vt[2][D * VS];

    int seq, head, qg;
    if (D >= 64 && units > 0) {
        if (!block_unit(a, gx, units, seq, head, qg)) return;
    } else {
        block_item(a, seq, head, qg);
    }
    const int start = a.offsets[seq];
    const int L = a.offsets[seq + 1] - start;
    const int nq = min(L, a.q_limit);
    const int q0 = qg * QROWS;
    if (q0 >= nq) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int H = a.H, ld = 3 * H;
    const f16 *kbase = a.qkv + (size_t)start * ld + H + head * D, *vbase = kbase + H;

    f16x8 qf[QT][D / 32];
    load_q<D, QT, ROPE>(a, start, L, q0 + wave * QT * 16, lane, qf, head);

    // Staging registers of one key block.
    f16x8 rk[NKI][ROPE ? 2 : 1], rv[NVI][2];
    auto load_kv = [&](int kb0) {
#pragma unroll
        for (int i = 0; i < NKI; ++i) {
            const int c = i * NT + tid;
            if (KI % NT == 0 || c < KI) {
                constexpr int PR = ROPE ? HCH : CPR;
                const int key = min(kb0 + c / PR, L - 1), ch = c % PR;
                const f16 *r = kbase + (size_t)key * ld + ch * 8;
                rk[i][0] = *(const f16x8 *)r;
                if constexpr (ROPE) rk[i][1] = *(const f16x8 *)(r + D / 2);
            }
        }
#pragma unroll
        for (int i = 0; i < NVI; ++i) {
            const int c = i * NT + tid;
            if (VI % NT == 0 || c < VI) {
                const int p = c / CPR, ch = c % CPR;
                rv[i][0] = *(const f16x8 *)(vbase + (size_t)min(kb0 + 2 * p, L - 1) * ld + ch * 8);
                rv[i][1] = *(const f16x8 *)(vbase + (size_t)min(kb0 + 2 * p + 1, L - 1) * ld + ch * 8);
            }
        }
    };
    auto store_kv = [&](int buf, int kb0) {
#pragma unroll
        for (int i = 0; i < NKI; ++i) {
            const int c = i * NT + tid;
            if (KI % NT == 0 || c < KI) {
                constexpr int PR = ROPE ? HCH : CPR;
                const int r = c / PR, ch = c % PR;
                if constexpr (ROPE) {
                    // rotateHalf on dims i = 8·ch + e and i + D/2 (model.go:705-712)
                    const int pos = min(kb0 + r, L - 1);
                    const float *cp = a.rope_cos + (size_t)pos * (D / 2) + ch * 8;
                    const float *sp = a.rope_sin + (size_t)pos * (D / 2) + ch * 8;
                    const f32x4 c0 = *(const f32x4 *)cp, c1 = *(const f32x4 *)(cp + 4);
                    const f32x4 s0 = *(const f32x4 *)sp, s1 = *(const f32x4 *)(sp + 4);
                    f16x8 lo, hi;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float cs = e < 4 ? c0[e] : c1[e - 4], sn = e < 4 ? s0[e] : s1[e - 4];
                        const float x1 = (float)rk[i][0][e], x2 = (float)rk[i][1][e];
                        lo[e] = (f16)rot(x1, x2, cs, sn, true);
                        hi[e] = (f16)rot(x2, x1, cs, sn, false);
                    }
                    *(f16x8 *)&Ks[buf][r * KS + ch * 8] = lo;
                    *(f16x8 *)&Ks[buf][r * KS + ch * 8 + D / 2] = hi;
                } else {
                    *(f16x8 *)&Ks[buf][r * KS + ch * 8] = rk[i][0];
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NVI; ++i) {
            const int c = i * NT + tid;
            if (VI % NT == 0 || c < VI) {
                const int p = c / CPR, ch = c % CPR;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    *(f16x2 *)&Vt[buf][(ch * 8 + j) * VS + 2 * p] = (f16x2){rv[i][0][j], rv[i][1][j]};
            }
        }
    };

    f32x4 o[QT][D / 16];
    float m_run[QT], l_run[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        m_run[qt] = -INFINITY;
        l_run[qt] = 0.f;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) o[qt][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    const float sl2 = a.scale_log2e;

    // One query tile against key block `buf` (kvalid valid keys from its
    // first).  MASK: the block has fewer than BK valid keys (only the last
    // can); a separate copy, so that full blocks carry no masking selects.
    auto qtile = [&](int qt, int buf, int kvalid, auto mask_t) {
        constexpr bool MASK = decltype(mask_t)::value;
        f32x4 s[NKT];
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int dk = 0; dk < D / 32; ++dk) {
                const f16x8 kf = *(const f16x8 *)&Ks[buf][(kt * 16 + (lane & 15)) * KS + dk * 32 + (lane >> 4) * 8];
                s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[qt][dk], s[kt], 0, 0, 0);
            }
            if constexpr (MASK) {  // the last key block: keys past the sequence
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (kt * 16 + (lane >> 4) * 4 + i >= kvalid) s[kt][i] = -INFINITY;
            }
            mx = fmaxf(mx, fmaxf(fmaxf(s[kt][0], s[kt][1]), fmaxf(s[kt][2], s[kt][3])));
        }
        mx = max_xor32(max_xor16(mx));
        const float m_new = fmaxf(m_run[qt], mx * sl2);  // log2-scaled running max
        const float corr = __builtin_amdgcn_exp2f(m_run[qt] - m_new);
        f16x8 pf[NC];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) pf[kt >> 1][(kt & 1) * 4 + i] = (f16)__builtin_amdgcn_exp2f(s[kt][i] * sl2 - m_new);
        const float psum = prob_sum<NC>(pf);  // the block's sum of the binary16 probabilities
        l_run[qt] = l_run[qt] * corr + psum;
        m_run[qt] = m_new;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) o[qt][t] *= corr;
        // Oᵀ += Vᵀ·Pᵀ over 32-key chunks; key slots {4g..4g+3, 16+4g..16+4g+3}, g = lane/16.
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
            for (int t = 0; t < D / 16; ++t) {
                const f16 *vrow = &Vt[buf][(t * 16 + (lane & 15)) * VS + c * 32 + (lane >> 4) * 4];
                const f16x4 lo = *(const f16x4 *)vrow;
                const f16x4 hi = *(const f16x4 *)(vrow + 16);
                const f16x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[qt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[c], o[qt][t], 0, 0, 0);
            }
        }
    };

    // Every key block but the last is full and has a successor, so the loop
    // body is one straight path (a branch between the full and the masked
    // copy inside it made the compiler shuffle the loop-carried registers,
    // ~56 moves per key block); the last block follows the loop.
    const int nkb = (L + BK - 1) / BK;
    load_kv(0);
    store_kv(0, 0);
    __syncthreads();
    for (int kb = 0; kb + 1 < nkb; ++kb) {
        const int kb0 = kb * BK, buf = kb & 1;
        load_kv(kb0 + BK);  // in flight while this block is multiplied
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
            if (q0 + (wave * QT + qt) * 16 < nq) qtile(qt, buf, BK, std::false_type{});  // wave-uniform
        // The other buffer was last read before the previous barrier.
        store_kv(buf ^ 1, kb0 + BK);
        __syncthreads();
    }
    {
        const int kb0 = (nkb - 1) * BK, buf = (nkb - 1) & 1;
        if (L - kb0 >= BK) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt)
                if (q0 + (wave * QT + qt) * 16 < nq) qtile(qt, buf, BK, std::false_type{});
        } else {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt)
                if (q0 + (wave * QT + qt) * 16 < nq) qtile(qt, buf, L - kb0, std::true_type{});
        }
    }

    // Lane owns O[query lane%16][dims t·16 + (lane/16)·4 .. +4] of each tile.
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int q = q0 + (wave * QT + qt) * 16 + (lane & 15);
        if (q >= nq) continue;
        const float inv = 1.0f / l_run[qt];
        const size_t orow = a.compact ? (size_t)seq : (size_t)(start + q);
#pragma unroll
        for (int t = 0; t < D / 16; ++t) {
            const int dim = t * 16 + (lane >> 4) * 4;
            const f32x4 v = o[qt][t] * inv;
            if (OUT_F32) {
                *(f32x4 *)((float *)a.out + orow * a.ldo + head * D + dim) = v;
            } else {
                const f16x4 h = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
                *(f16x4 *)((f16 *)a.out + orow * a.ldo + head * D + dim) = h;
            }
        }
    }
}

template <int D, int WAVES, int QT>
hipError_t launch_long(const AttnArgs &a, int nseq, int max_len, bool out_f32, bool rope, hipStream_t s) {
    constexpr int QROWS = 16 * QT * WAVES;
    const int qmax = min(max_len, a.q_limit);
    const int gx = (qmax + QROWS - 1) / QROWS;
    // D ≥ 64: (sequence, head) units dealt to the XCDs (block_unit) while the
    // 1-D grid's work-items fit 32 bits; else (units = 0) block_item's
    // (query group, head, sequence) grid.
    const long nblk = (long)gx * (((long)a.H / a.d * nseq + 7) / 8 * 8);
    const int units = D >= 64 && nblk * (WAVES * 64) < (1l << 32) ? a.H / a.d * nseq : 0;
    dim3 grid = units ? dim3((unsigned)nblk) : dim3(gx, a.H / a.d, nseq);
    dim3 block(WAVES * 64);
    if (out_f32) {
        if (rope) hipLaunchKernelGGL((attn_long_kernel<D, WAVES, QT, true, true>), grid, block, 0, s, a, gx, units);
        else hipLaunchKernelGGL((attn_long_kernel<D, WAVES, QT, true, false>), grid, block, 0, s, a, gx, units);
    } else {
        if (rope) hipLaunchKernelGGL((attn_long_kernel<D, WAVES, QT, false, true>), grid, block, 0, s, a, gx, units);
        else hipLaunchKernelGGL((attn_long_kernel<D, WAVES, QT, false, false>), grid, block, 0, s, a, gx, units);
    }
    return hipGetLastError();
}

template <int D, int WAVES, int QT, int KBLK, bool ONE>
hipError_t launch_d(const AttnArgs &a, int nseq, int max_len, bool out_f32, bool rope, hipStream_t s) {
    constexpr int QROWS = 16 * QT * WAVES;
    if (ONE && max_len > KBLK) return hipErrorInvalidValue;  // one key block must hold every sequence
    const int qmax = min(max_len, a.q_limit);
    dim3 grid((qmax + QROWS - 1) / QROWS, a.H / a.d, nseq);
    dim3 block(WAVES * 64);
    if (out_f32) {
        if (rope) hipLaunchKernelGGL((attn_kernel<D, WAVES, QT, KBLK, true, true, ONE>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((attn_kernel<D, WAVES, QT, KBLK, true, false, ONE>), grid, block, 0, s, a);
    } else {
        if (rope) hipLaunchKernelGGL((attn_kernel<D, WAVES, QT, KBLK, false, true, ONE>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((attn_kernel<D, WAVES, QT, KBLK, false, false, ONE>), grid, block, 0, s, a);
    }
    return hipGetLastError();
}

static_assert(fh::ATTN_ONE_BLOCK_KEYS == 128, "the one-block kernels stage 128 keys");

template <int D>
hipError_t launch_w(const AttnArgs &a, int nseq, int max_len, bool out_f32, bool rope, hipStream_t s) {
    // CLS row only: one wave per (sequence, head).
    if (a.q_limit <= 16) {
        if (max_len <= fh::ATTN_ONE_BLOCK_KEYS) return launch_d<D, 1, 1, 128, true>(a, nseq, max_len, out_f32, rope, s);
        return launch_d<D, 1, 1, 64, false>(a, nseq, max_len, out_f32, rope, s);
    }
    // Up to 64 tokens: 64 query rows per block (2 waves x 2 tiles); smaller
    // blocks keep more of them resident (18 us vs 24 us for 512 sequences
    // of 16..64 tokens at 12 heads of 32).
    if (max_len <= 64) return launch_d<D, 2, 2, 128, true>(a, nseq, max_len, out_f32, rope, s);
    // Up to 128 tokens: one block covers every query and stages K/V once.
    if (max_len <= fh::ATTN_ONE_BLOCK_KEYS) return launch_d<D, 4, 2, 128, true>(a, nseq, max_len, out_f32, rope, s);
    if (a.d == D && long_pipeline()) {
        // Same per-query arithmetic (same bits) in either shape.  Up to 1024
        // tokens, 256-query blocks of 8 waves (BERT-base, 512 tokens: 2.59 →
        // 2.40 ms per step against 4 × 2); beyond, three query tiles per wave
        // share each K/V fragment read and key-block barrier (nomic-bert,
        // 540..2021 tokens: 3.08 → 2.83 ms against 4 × 2, while 8 × 2 gains
        // nothing there).
        // At head width 32, 8 × 2 measured no faster than 4 × 2 (bge-small,
        // a mixed batch of 2..512 tokens).
        if (D < 64) return launch_long<D, 4, 2>(a, nseq, max_len, out_f32, rope, s);
        if (max_len > ATTN_LONG_SPLIT) return launch_long<D, 4, 3>(a, nseq, max_len, out_f32, rope, s);
        return launch_long<D, 8, 2>(a, nseq, max_len, out_f32, rope, s);
    }
    return launch_d<D, 4, 1, 64, false>(a, nseq, max_len, out_f32, rope, s);
}

}  // namespace

namespace fh {
bool rope_qk_ok(int H, int d) { return d > 0 && H % d == 0 && (d / 2) % 8 == 0; }

hipError_t rope_qk(f16 *qkv, const int32_t *offsets, int nseq, int max_len, int H, int d, const float *cos_t,
                   const float *sin_t, hipStream_t s) {
    if (!rope_qk_ok(H, d)) return hipErrorInvalidValue;
    if (nseq <= 0 || max_len <= 0) return hipSuccess;
    const long units = (long)max_len * 2 * (H / d) * (d / 16);
    hipLaunchKernelGGL(rope_qk_kernel, dim3((unsigned)((units + 255) / 256), nseq), dim3(256), 0, s, qkv, offsets, H, d,
                       cos_t, sin_t);
    return hipGetLastError();
}

hipError_t attention(const AttnArgs &a, int nseq, int max_len, bool out_f32, hipStream_t s) {
    if (nseq <= 0 || max_len <= 0) return hipSuccess;
    const bool rope = a.rope_cos != nullptr;
    if (a.d <= 32) return launch_w<32>(a, nseq, max_len, out_f32, rope, s);
    if (a.d <= 64) return launch_w<64>(a, nseq, max_len, out_f32, rope, s);
    if (a.d <= 128) return launch_w<128>(a, nseq, max_len, out_f32, rope, s);
    return hipErrorInvalidValue;
}
}  // namespace fh
