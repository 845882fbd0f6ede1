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
// Tiling: 128×128 block tile, 256 threads = 4 waves in 2×2, 64×64 per wave
// (4×4 MFMA tiles), 64-element (f16) / 128-byte (i8) K slices staged
// through double-buffered LDS with one barrier per K slice.  The MFMA is
// issued with the weight fragment as the A operand, so each lane ends up
// holding four consecutive output columns of one row: epilogue stores are
// 8/16-byte vectors, and the SwiGLU up/gate pair (interleaved in 16-row
// blocks at load) lands in the same lane.
#include "fh_common.h"

namespace {

constexpr int BM = 128, BN = 128, NT = 256;
constexpr int KB = 128;            // bytes of K per slice (64 f16 or 128 i8)
constexpr int LDS_ROW = KB + 16;   // bytes; +16 staggers rows across LDS banks

__device__ __forceinline__ float gelu_erf(float x) {
    // 0.5·x·(1 + erf(x/√2)) written through erfc so both tails stay accurate.
    return 0.5f * x * erfcf(-x * 0.70710678118654752f);
}
__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

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

template <int ACT, bool OUT_F32>
__device__ __forceinline__ void epilogue_store(const GemmArgs &g, int row, int col, f32x4 v,
                                               f32x4 gate) {
    if (ACT == fh::ACT_SWIGLU) {
        // col is the packed up-column; output column folds the 16-row interleave.
        const int ocol = ((col >> 5) << 4) + (col & 15);
        if (g.bias) {
            const f32x4 bu = *(const f32x4 *)(g.bias + col);
            const f32x4 bg = *(const f32x4 *)(g.bias + col + 16);
            v += bu;
            gate += bg;
        }
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = v[i] * silu(gate[i]);
        if (OUT_F32) {
            *(f32x4 *)((float *)g.C + (size_t)row * g.ldc + ocol) = o;
        } else {
            f16x4 h = {(f16)o[0], (f16)o[1], (f16)o[2], (f16)o[3]};
            *(f16x4 *)((f16 *)g.C + (size_t)row * g.ldc + ocol) = h;
        }
        return;
    }
    if (g.bias) v += *(const f32x4 *)(g.bias + col);
    if (ACT == fh::ACT_GELU) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = gelu_erf(v[i]);
    }
    if (g.resid) v += *(const f32x4 *)(g.resid + (size_t)row * g.ldr + col);
    if (OUT_F32) {
        *(f32x4 *)((float *)g.C + (size_t)row * g.ldc + col) = v;
    } else {
        f16x4 h = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
        *(f16x4 *)((f16 *)g.C + (size_t)row * g.ldc + col) = h;
    }
}

// One kernel body for both element types.  ELT = bytes per element of A/B.
template <bool I8, int ACT, bool OUT_F32>
__global__ __launch_bounds__(NT, 2) void gemm_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) uint8_t As[2][BM * LDS_ROW];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BN * LDS_ROW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int mt, nt;
    tile_coords(mt, nt);
    const int m0 = mt * BM, n0 = nt * BN;
    constexpr int ESZ = I8 ? 1 : 2;
    const int kbytes = g.K * ESZ;
    const uint8_t *A = (const uint8_t *)g.A;
    const uint8_t *B = (const uint8_t *)g.B;
    const size_t lda = (size_t)g.lda * ESZ, ldb = (size_t)g.ldb * ESZ;

    // Each thread moves 4 sixteen-byte chunks of A and of B per K slice:
    // chunk c = tid + i·256 covers row c/8, bytes (c%8)·16 of the slice.
    i32x4 ra[4], rb[4];
    const i32x4 zero = {0, 0, 0, 0};
    auto gload = [&](int kb0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + i * NT, r = c >> 3, kb = kb0 + (c & 7) * 16;
            const int ar = min(m0 + r, g.M - 1), br = min(n0 + r, g.N - 1);
            ra[i] = kb < kbytes ? *(const i32x4 *)(A + ar * lda + kb) : zero;
            rb[i] = kb < kbytes ? *(const i32x4 *)(B + br * ldb + kb) : zero;
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + i * NT, r = c >> 3, cb = (c & 7) * 16;
            *(i32x4 *)&As[buf][r * LDS_ROW + cb] = ra[i];
            *(i32x4 *)&Bs[buf][r * LDS_ROW + cb] = rb[i];
        }
    };

    f32x4 acc[4][4];
    i32x4 iacc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            acc[a][b] = (f32x4){0.f, 0.f, 0.f, 0.f};
            iacc[a][b] = zero;
        }

    const int nk = (kbytes + KB - 1) / KB;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * KB);
#pragma unroll
        for (int kk = 0; kk < KB; kk += 64) {  // 64 bytes of K per MFMA step
            i32x4 af[4], bf[4];
            const int kofs = kk + (lane >> 4) * 16;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                af[t] = *(const i32x4 *)&As[cur][(wm * 64 + t * 16 + (lane & 15)) * LDS_ROW + kofs];
                bf[t] = *(const i32x4 *)&Bs[cur][(wn * 64 + t * 16 + (lane & 15)) * LDS_ROW + kofs];
            }
#pragma unroll
            for (int tn = 0; tn < 4; ++tn)
#pragma unroll
                for (int tm = 0; tm < 4; ++tm) {
                    if (I8) {
                        iacc[tn][tm] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[tn], af[tm], iacc[tn][tm],
                                                                            0, 0, 0);
                    } else {
                        acc[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(f16x8, bf[tn]), __builtin_bit_cast(f16x8, af[tm]),
                            acc[tn][tm], 0, 0, 0);
                    }
                }
        }
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }

    // Lane holds C[row][col .. col+3] for row = tile_m + lane%16,
    // col = tile_n + (lane/16)·4.
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
        const int row = m0 + wm * 64 + tm * 16 + (lane & 15);
        if (row >= g.M) continue;
        float sa = 0.f;
        if (I8) sa = g.a_scale[row];
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
            if (ACT == fh::ACT_SWIGLU && (tn & 1)) continue;
            const int col = n0 + wn * 64 + tn * 16 + (lane >> 4) * 4;
            if (col >= g.N) continue;
            f32x4 v, gate = {0.f, 0.f, 0.f, 0.f};
            if (I8) {
                const f32x4 sb = *(const f32x4 *)(g.b_scale + col);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    v[i] = __fmul_rn((float)iacc[tn][tm][i], __fmul_rn(sa, sb[i]));
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
            epilogue_store<ACT, OUT_F32>(g, row, col, v, gate);
        }
    }
}

template <bool I8>
hipError_t launch(const GemmArgs &g, int act, bool out_f32, hipStream_t s) {
    if (g.M <= 0) return hipSuccess;
    dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM);
    dim3 block(NT);
#define FH_GEMM_CASE(ACTV, F32)                                                              \
    if (act == ACTV && out_f32 == F32) {                                                    \
        hipLaunchKernelGGL((gemm_kernel<I8, ACTV, F32>), grid, block, 0, s, g);            \
        return hipGetLastError();                                                           \
    }
    FH_GEMM_CASE(fh::ACT_NONE, false)
    FH_GEMM_CASE(fh::ACT_NONE, true)
    FH_GEMM_CASE(fh::ACT_GELU, false)
    FH_GEMM_CASE(fh::ACT_GELU, true)
    FH_GEMM_CASE(fh::ACT_SWIGLU, false)
    FH_GEMM_CASE(fh::ACT_SWIGLU, true)
#undef FH_GEMM_CASE
    return hipErrorInvalidValue;
}

}  // namespace

namespace fh {
hipError_t gemm_f16(const GemmArgs &a, int act, bool out_f32, hipStream_t s) {
    return launch<false>(a, act, out_f32, s);
}
hipError_t gemm_i8(const GemmArgs &a, int act, bool out_f32, hipStream_t s) {
    return launch<true>(a, act, out_f32, s);
}
}  // namespace fh
