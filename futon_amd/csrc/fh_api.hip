// Host orchestration behind include/futon_hip.h: weight upload, workspace,
// per-batch kernel schedule, cancellation checkpoints, profiling.
//
// The schedule is the reference forward (native/model.go:346-457,
// :550-635) over a packed batch:
//   embed+LN → per layer { QKV GEMM → attention → out GEMM(+bias+residual)
//   → LN → FFN GEMM(+bias, GELU | SwiGLU) → fc2 GEMM(+bias+residual) → LN }
//   → pool → Matryoshka → L2.
// With CLS pooling the last layer computes only each sequence's row 0 after
// the attention (model.go:403-410): the CLS rows are gathered into a compact
// [nseq, H] buffer and the out/FFN GEMMs run with M = nseq.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/futon_hip.h"
#include "../../include/futon_hip_ops.h"
#include "fh_common.h"
#include "host/host_common.h"

// Device memory of fh_encode_device_noalloc: every buffer of a forward
// beyond its inputs and outputs (the workspace fh_encode_device allocates),
// in one array per device, held until the process ends.  Host code never
// uses the name itself: fh_model_create looks up each device's address
// (hipGetSymbolAddress) once, and the entry point passes that address on.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

using fh::fail;

// Per device: the scratch array's device address, and the event that marks
// the end of the last forward that used it (later calls queue behind it,
// whatever stream or model they come from).
constexpr int kMaxDevices = 64;
struct DevScratch {
    void *ptr = nullptr;
    hipEvent_t done = nullptr;
    bool used = false;
};
std::mutex g_scratch_mu;
DevScratch g_scratch[kMaxDevices];

// Once per device, with that device current.
int init_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return fail(FH_ENODEV, "device %d beyond %d", device, kMaxDevices);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    DevScratch &d = g_scratch[device];
    if (d.ptr) return FH_OK;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return fail(FH_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    e = hipEventCreateWithFlags(&d.done, hipEventDisableTiming);
    if (e != hipSuccess) return fail(FH_EHIP, "hipEventCreate: %s", hipGetErrorString(e));
    d.ptr = p;
    return FH_OK;
}

#define HIPCHK(expr)                                                                       \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess) return fail(FH_EHIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

// Exact binary16 → binary32 (native/safetensors.go:266-289).
float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31, exp = (h >> 10) & 0x1f, mant = h & 0x3ff, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            uint32_t e = 127 - 15 + 1;
            while (!(mant & 0x400)) {
                mant <<= 1;
                e--;
            }
            bits = sign | e << 23 | (mant & 0x3ff) << 13;
        }
    } else if (exp == 0x1f) {
        bits = sign | 0xffu << 23 | mant << 13;
    } else {
        bits = sign | (exp + 127 - 15) << 23 | mant << 13;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// binary32 → binary16, round to nearest even (native/safetensors.go:226-262).
uint16_t f32_to_f16(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    uint16_t sign = (uint16_t)(b >> 16) & 0x8000;
    int32_t exp32 = (int32_t)(b >> 23 & 0xff), exp = exp32 - 127 + 15;
    uint32_t mant = b & 0x7fffff;
    if (exp32 == 0xff) return mant ? (sign | 0x7e00) : (sign | 0x7c00);
    if (exp >= 0x1f) return sign | 0x7c00;
    if (exp <= 0) {
        if (exp < -10) return sign;
        mant |= 0x800000;
        uint32_t shift = (uint32_t)(14 - exp), half = mant >> shift, rem = mant & ((1u << shift) - 1),
                 hw = 1u << (shift - 1);
        if (rem > hw || (rem == hw && (half & 1))) half++;
        return sign | (uint16_t)half;
    }
    uint16_t half = (uint16_t)((uint32_t)exp << 10 | (mant >> 13));
    uint32_t rem = mant & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (half & 1))) half++;
    return sign | half;
}

// Per-row absmax int8 quantization (native/quant.go:42-70); float64 rounding
// half away from zero like math.Round.
float quantize_row_q8(int8_t *dst, const float *src, int n) {
    float amax = 0.f;
    for (int i = 0; i < n; i++) amax = std::max(amax, std::fabs(src[i]));
    if (amax == 0.f) {
        memset(dst, 0, (size_t)n);
        return 0.f;
    }
    const float scale = amax / 127.0f;
    const double inv = 127.0 / (double)amax;
    for (int i = 0; i < n; i++) {
        double q = std::round((double)src[i] * inv);
        q = std::min(127.0, std::max(-127.0, q));
        dst[i] = (int8_t)q;
    }
    return scale;
}

struct DevMat {
    void *w = nullptr;       // f16 [n,k] or i8 [n,k]
    float *scale = nullptr;  // i8: [n]
    int n = 0, k = 0;
    void *wr = nullptr;      // f16 copy with rows in fh::ring_pack_row order for fh::gemm_ring, or null
    void *wm = nullptr;      // f16 fragment-ordered copy for fh::mlp (fc1: mlp_w1_unit, fc2: mlp_w2_unit), or null
};

// The persistent ring GEMM pays off once its tiles cover about half the
// CUs; fewer rows (small batches, the CLS-pooled last layer) run on the
// tiled GEMM's smaller tiles with the natural-order copy.  The ring also
// addresses its operands with 32-bit buffer offsets: a problem whose rows
// overflow them (gemm_ring_ok) runs on the 64-bit-indexed tiled GEMM, with
// the same bits.
bool use_ring(const DevMat &w, const GemmArgs &g, int act, bool out_f32, int ln) {
    if (!w.wr || !fh::gemm_ring_worth(g.M, w.n)) return false;
    if (act == fh::ACT_NONE && !out_f32 && g.resid_h && !g.resid) act = fh::ACT_RES16;  // as gemm_ring does
    return fh::gemm_ring_ok(g, act, out_f32, ln);
}

struct DevLayer {
    DevMat qkv, out, ffn1, fc2;  // ffn1 = fc1, or fc1|gate interleaved in 16-row blocks (SwiGLU)
    float *qkv_b = nullptr, *out_b = nullptr, *ffn1_b = nullptr, *fc2_b = nullptr;
    float *n1w = nullptr, *n1b = nullptr, *n2w = nullptr, *n2b = nullptr;
    // LayerNorm folding (binary16 path): qkv/ffn1 weights are stored scaled by
    // the γ of the LayerNorm feeding them; c1 = row sums of those stored
    // weights, c2 = W·β + bias (float64 sums).
    float *qkv_c1 = nullptr, *qkv_c2 = nullptr, *ffn1_c1 = nullptr, *ffn1_c2 = nullptr;
};

enum KClass {
    K_EMBED, K_GEMM_QKV, K_ATTN, K_GEMM_OUT, K_LN, K_GEMM_FFN1, K_GEMM_FC2, K_QUANT, K_GATHER, K_POOL,
    K_CLS_TAIL,  // last CLS layer: attention for row 0, the CLS-row gather, statistics and norms (its GEMMs
                 // count in the GEMM classes)
    K_STATS,     // row statistics for the folded LayerNorms
    K_MLP,       // fused FFN1 → GELU → FC2 (fh::mlp)
    K_NCLASS
};
const char *kClassNames[K_NCLASS] = {"embed_ln",  "gemm_qkv", "attention", "gemm_out",
                                     "layer_norm", "gemm_ffn1", "gemm_fc2", "quantize_rows",
                                     "gather_cls", "pool_l2",    "cls_last_layer", "row_stats",
                                     "mlp_fused"};

struct ProfPending {
    int cls;
    hipEvent_t a, b;
    double flops, bytes;
};

}  // namespace

struct fh_model {
    fh_config cfg{};
    int device = 0, hd = 0, eff_max = 0;
    bool lnfold = false;  // LayerNorms folded into the GEMMs (binary16 path)
    // Q and K rotated by rope_qk before attention (RoPE packs whose head width
    // it covers); FUTON_ROPE_QK=0 leaves the rotation inside the attention
    // kernels (diagnostics: the same bits either way).
    bool rope_pre = false;
    // Pooling takes the last hidden state un-normalized and applies its
    // LayerNorm itself (mean: inside the segment sums, fh::ln_pool; CLS: on
    // the compact rows, fh::ln_cls_pool), for the widths those kernels cover;
    // FUTON_LN_POOL=0 keeps the LayerNorm and the pooling apart (diagnostics;
    // for mean pooling the segment sums are then added in another order).
    bool ln_pool = false;
    // The embedding kernel also writes the first layer's row statistics
    // (binary16 folded path; FUTON_EMBED_STATS=0 leaves them to row_stats:
    // diagnostics, the same bits).
    bool embed_stats = false;
    hipStream_t stream = nullptr;
    float *word = nullptr, *pos = nullptr, *type0 = nullptr, *emb_w = nullptr, *emb_b = nullptr;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    std::vector<DevLayer> layers;
    std::vector<void *> allocs;
    int64_t weight_bytes = 0;

    // Workspace, grown on demand (capacity in tokens / sequences).
    int cap_tokens = 0, cap_seqs = 0;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    float *x32 = nullptr, *y32 = nullptr, *xc32 = nullptr;
    float *pool_part = nullptr;  // mean pooling's segment sums
    f16 *x16 = nullptr, *qkv = nullptr, *xc16 = nullptr;
    void *attn = nullptr, *attnc = nullptr, *hbuf = nullptr;
    int8_t *xq = nullptr;
    float *xs = nullptr;
    f32x2 *sA = nullptr, *sB = nullptr, *sAc = nullptr, *sBc = nullptr;  // per-row (mean, rstd)
    f16 *yBc = nullptr;
    // fh_encode's batch I/O (ids in schedule order, per-chunk offsets, the
    // vectors): device buffer and pinned host staging of the same layout.
    void *io = nullptr;
    size_t io_bytes = 0;
    void *pin = nullptr;
    size_t pin_bytes = 0;
    int chunk_tokens = 1 << 18;  // most tokens one fh_encode chunk runs in one forward
    bool schedule = true;        // sort fh_encode batches and split attention by class (FUTON_SCHEDULE=0: batch
                                 // order, one attention launch sized by the longest sequence; for comparison)
    // Every forward is ordered after the previous one, whatever stream each
    // ran on: done_ev is recorded at the end of each forward (done_stream is
    // where), and the next forward's stream waits on it.  Synchronizing
    // done_ev therefore drains every earlier use of the workspace.
    hipEvent_t done_ev = nullptr;
    hipStream_t done_stream = nullptr;

    std::mutex mu;
    int cancel_after = -1;
    bool prof = false;
    std::vector<ProfPending> pending;
    std::vector<hipEvent_t> event_pool;
    double prof_ms[K_NCLASS] = {}, prof_flops[K_NCLASS] = {}, prof_bytes[K_NCLASS] = {};
    int64_t prof_launches[K_NCLASS] = {};
};

namespace {

template <class T>
int dev_alloc(fh_model *m, T **p, size_t bytes) {
    void *q = nullptr;
    hipError_t e = hipMalloc(&q, std::max<size_t>(bytes, 256));
    if (e != hipSuccess) return fail(FH_ENOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    m->allocs.push_back(q);
    m->weight_bytes += (int64_t)bytes;
    *p = (T *)q;
    return FH_OK;
}

template <class T>
int upload(fh_model *m, T **p, const void *host, size_t bytes) {
    int rc = dev_alloc(m, p, bytes);
    if (rc) return rc;
    HIPCHK(hipMemcpy(*p, host, bytes, hipMemcpyHostToDevice));
    return FH_OK;
}

struct TensorView {
    const fh_tensor *t = nullptr;
    int64_t numel() const {
        int64_t n = 1;
        for (int i = 0; i < t->rank; i++) n *= t->shape[i];
        return n;
    }
    // Element i as float32 (f16 converted exactly).
    void to_f32(std::vector<float> &dst) const {
        const int64_t n = numel();
        dst.resize((size_t)n);
        if (t->dtype == FH_DTYPE_F32) {
            memcpy(dst.data(), t->data, (size_t)n * 4);
        } else {
            const uint16_t *s = (const uint16_t *)t->data;
            for (int64_t i = 0; i < n; i++) dst[(size_t)i] = f16_to_f32(s[i]);
        }
    }
};

struct Loader {
    fh_model *m;
    const fh_tensor *ts;
    int n;
    std::vector<bool> used;
    std::string model_id = "pack";

    int find(const std::string &name) const {
        for (int i = 0; i < n; i++)
            if (ts[i].name && name == ts[i].name) return i;
        return -1;
    }
    // needT (native/model.go:143-158): presence, rank and shape.
    int need(const std::string &name, std::initializer_list<int64_t> shape, TensorView &tv,
             bool optional = false, bool *present = nullptr) {
        const int i = find(name);
        if (present) *present = i >= 0;
        if (i < 0) {
            if (optional) return FH_OK;
            return fail(FH_EINVAL, "pack %s: missing tensor \"%s\"", model_id.c_str(), name.c_str());
        }
        used[(size_t)i] = true;
        const fh_tensor &t = ts[i];
        if (t.rank != (int)shape.size())
            return fail(FH_EINVAL, "pack %s: tensor \"%s\" rank %d, want %d", model_id.c_str(), name.c_str(),
                        t.rank, (int)shape.size());
        int j = 0;
        for (int64_t d : shape) {
            if (t.shape[j] != d)
                return fail(FH_EINVAL, "pack %s: tensor \"%s\" dim %d is %lld, want %lld", model_id.c_str(),
                            name.c_str(), j, (long long)t.shape[j], (long long)d);
            j++;
        }
        if (t.dtype != FH_DTYPE_F32 && t.dtype != FH_DTYPE_F16)
            return fail(FH_EINVAL, "pack %s: tensor \"%s\" has unsupported dtype %d", model_id.c_str(),
                        name.c_str(), t.dtype);
        if (!t.data) return fail(FH_EINVAL, "pack %s: tensor \"%s\" has no data", model_id.c_str(), name.c_str());
        tv.t = &t;
        return FH_OK;
    }
    int vec_f32(const std::string &name, int64_t len, float **dst, bool optional = false) {
        TensorView tv;
        bool present = true;
        int rc = need(name, {len}, tv, optional, &present);
        if (rc || !present) return rc;
        std::vector<float> h;
        tv.to_f32(h);
        return upload(m, dst, h.data(), h.size() * 4);
    }
    int vec_host(const std::string &name, int64_t len, std::vector<float> &h, bool optional = false) {
        TensorView tv;
        bool present = true;
        int rc = need(name, {len}, tv, optional, &present);
        if (rc) return rc;
        if (!present) {
            h.clear();
            return FH_OK;
        }
        tv.to_f32(h);
        return FH_OK;
    }
    int mat_f32(const std::string &name, int64_t r, int64_t c, float **dst) {
        TensorView tv;
        int rc = need(name, {r, c}, tv);
        if (rc) return rc;
        std::vector<float> h;
        tv.to_f32(h);
        return upload(m, dst, h.data(), h.size() * 4);
    }
    int mat_host(const std::string &name, int64_t r, int64_t c, std::vector<float> &h) {
        TensorView tv;
        int rc = need(name, {r, c}, tv);
        if (rc) return rc;
        tv.to_f32(h);
        return FH_OK;
    }
};

// LayerNorm folding of a GEMM fed by LN(y) = (y − mean)·rstd·γ + β:
// x·Wᵀ + b = rstd·(y·W'ᵀ − mean·c1) + c2 with W' = f16(W·diag(γ)),
// c1[n] = Σ_k W'[n,k] (of the stored binary16 values, so the mean term
// cancels exactly what y·W'ᵀ contains) and c2[n] = Σ_k W[n,k]·β[k] + b[n].
void fold_ln(std::vector<float> &w, int n, int k, const std::vector<float> &g, const std::vector<float> &beta,
             const std::vector<float> &bias, std::vector<float> &c1, std::vector<float> &c2) {
    c1.assign((size_t)n, 0.f);
    c2.assign((size_t)n, 0.f);
    for (int r = 0; r < n; r++) {
        float *row = &w[(size_t)r * k];
        double s1 = 0.0, s2 = bias.empty() ? 0.0 : (double)bias[(size_t)r];
        for (int j = 0; j < k; j++) {
            s2 += (double)row[j] * (double)beta[(size_t)j];
            row[j] = f16_to_f32(f32_to_f16(row[j] * g[(size_t)j]));
            s1 += (double)row[j];
        }
        c1[(size_t)r] = (float)s1;
        c2[(size_t)r] = (float)s2;
    }
}

// Uploads an [n,k] float matrix as f16 (RNE) or as Q8 codes + scales; with
// ring, also as f16 rows in fh::ring_pack_row order for fh::gemm_ring; with
// mlp_kind 1 or 2, also as the fragment-ordered fc1 or fc2 copy for fh::mlp.
int upload_mat(fh_model *m, DevMat &d, const std::vector<float> &w, int n, int k, bool q8, bool ring = false,
               int mlp_kind = 0) {
    d.n = n;
    d.k = k;
    if (mlp_kind && !q8) {
        std::vector<uint16_t> h(w.size());
        for (long u = 0; u < (long)n * k / 8; u++) {
            int row, col;
            if (mlp_kind == 1) fh::mlp_w1_unit(u, k, row, col);
            else fh::mlp_w2_unit(u, k, row, col);
            for (int e = 0; e < 8; e++) h[(size_t)u * 8 + e] = f32_to_f16(w[(size_t)row * k + col + e]);
        }
        const int rc = upload(m, (uint16_t **)&d.wm, h.data(), h.size() * 2);
        if (rc) return rc;
    }
    if (ring && !q8) {
        std::vector<uint16_t> h(w.size());
        for (int r = 0; r < n; r++) {
            const float *src = &w[(size_t)fh::ring_pack_row(r) * k];
            for (int j = 0; j < k; j++) h[(size_t)r * k + j] = f32_to_f16(src[j]);
        }
        const int rc = upload(m, (uint16_t **)&d.wr, h.data(), h.size() * 2);
        if (rc) return rc;
    }
    if (q8) {
        std::vector<int8_t> codes((size_t)n * k);
        std::vector<float> sc((size_t)n);
        for (int j = 0; j < n; j++) sc[(size_t)j] = quantize_row_q8(&codes[(size_t)j * k], &w[(size_t)j * k], k);
        int rc = upload(m, (int8_t **)&d.w, codes.data(), codes.size());
        if (rc) return rc;
        if (ring) {  // the codes' rows in ring_pack_row order; scales stay by output column
            std::vector<int8_t> pc(codes.size());
            for (int r = 0; r < n; r++)
                std::copy_n(&codes[(size_t)fh::ring_pack_row(r) * k], k, &pc[(size_t)r * k]);
            if ((rc = upload(m, (int8_t **)&d.wr, pc.data(), pc.size()))) return rc;
        }
        return upload(m, &d.scale, sc.data(), sc.size() * 4);
    }
    std::vector<uint16_t> h(w.size());
    for (size_t i = 0; i < w.size(); i++) h[i] = f32_to_f16(w[i]);
    return upload(m, (uint16_t **)&d.w, h.data(), h.size() * 2);
}

// SwiGLU packing: packed row r → fc1 row 16·(r/32) + r%32 when r%32 < 16,
// else gate row 16·(r/32) + r%32 − 16.
void interleave16(const std::vector<float> &up, const std::vector<float> &gate, int I, int k,
                  std::vector<float> &dst) {
    dst.resize((size_t)2 * I * k);
    for (int r = 0; r < 2 * I; r++) {
        const int blk = r / 32, w = r % 32;
        const std::vector<float> &src = w < 16 ? up : gate;
        const int sr = 16 * blk + (w % 16);
        memcpy(&dst[(size_t)r * k], &src[(size_t)sr * k], (size_t)k * 4);
    }
}

int eff_max_len(const fh_config &c) {
    return (c.max_trained_positions > 0 && c.max_trained_positions < c.max_seq_len) ? c.max_trained_positions
                                                                                     : c.max_seq_len;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Waits for every forward enqueued so far on any stream (they are chained
// through done_ev) and for the model's own stream.
hipError_t drain(fh_model *m) {
    hipError_t e = hipSuccess;
    if (m->done_stream) e = hipEventSynchronize(m->done_ev);
    const hipError_t e2 = hipStreamSynchronize(m->stream);
    return e != hipSuccess ? e : e2;
}

// A forward on stream s starts after the previous forward ends (which may
// have run on another stream) ...
int begin_on(fh_model *m, hipStream_t s) {
    if (m->done_stream && !(s == m->stream && m->done_stream == m->stream))
        HIPCHK(hipStreamWaitEvent(s, m->done_ev, 0));
    return FH_OK;
}
// ... and marks its own end.
int end_on(fh_model *m, hipStream_t s) {
    HIPCHK(hipEventRecord(m->done_ev, s));
    m->done_stream = s;
    return FH_OK;
}

// fh_encode's I/O buffers, device and pinned host, `bytes` each.
int ensure_io(fh_model *m, size_t bytes) {
    if (bytes <= m->io_bytes && bytes <= m->pin_bytes) return FH_OK;
    HIPCHK(drain(m));
    if (m->io) HIPCHK(hipFree(m->io));
    if (m->pin) HIPCHK(hipHostFree(m->pin));
    m->io = m->pin = nullptr;
    m->io_bytes = m->pin_bytes = 0;
    hipError_t e = hipMalloc(&m->io, bytes);
    if (e != hipSuccess) return fail(FH_ENOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    e = hipHostMalloc(&m->pin, bytes, hipHostMallocDefault);
    if (e != hipSuccess) return fail(FH_ENOMEM, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(e));
    m->io_bytes = m->pin_bytes = bytes;
    return FH_OK;
}

// The workspace for T tokens and S sequences: each of the model's buffer
// pointers with its size, in layout order (regions 256-byte aligned).
// (A fixed-capacity list, so laying out a workspace allocates nothing.)
struct WsPlan {
    std::pair<void **, size_t> e[20];
    int n = 0;
    const std::pair<void **, size_t> *begin() const { return e; }
    const std::pair<void **, size_t> *end() const { return e + n; }
    void push_back(std::pair<void **, size_t> p) { e[n++] = p; }
};
bool rope_pre(const fh_model *m) { return m->rope_pre; }


WsPlan workspace_plan(fh_model *m, int T, int S) {
    const size_t H = (size_t)m->cfg.hidden_size, I = (size_t)m->cfg.intermediate_size;
    const bool q8 = m->cfg.q8 != 0;
    const size_t hsz = q8 ? 4 : 2;  // FFN hidden / attention output element size
    WsPlan plan;
    for (auto p : std::initializer_list<std::pair<void **, size_t>>{
        {(void **)&m->x32, (size_t)T * H * 4},        {(void **)&m->x16, (size_t)T * H * 2},
        {(void **)&m->qkv, (size_t)T * 3 * H * 2},    {(void **)&m->attn, (size_t)T * H * hsz},
        {(void **)&m->y32, (size_t)T * H * 4},        {(void **)&m->hbuf, (size_t)T * I * hsz},
        {(void **)&m->xc32, (size_t)S * H * 4},       {(void **)&m->xc16, (size_t)S * H * 2},
        {(void **)&m->attnc, (size_t)S * H * hsz},
        {(void **)&m->sA, (size_t)T * 8},             {(void **)&m->sB, (size_t)T * 8},
        {(void **)&m->sAc, (size_t)S * 8},            {(void **)&m->sBc, (size_t)S * 8},
        {(void **)&m->yBc, (size_t)S * H * 2},
        {(void **)&m->pool_part, (size_t)fh::pool_part_rows(T, S) * H * 4},
    })
        plan.push_back(p);
    if (q8) {
        plan.push_back({(void **)&m->xq, (size_t)T * std::max(H, I)});
        plan.push_back({(void **)&m->xs, (size_t)T * 4});
    }
    return plan;
}

size_t workspace_bytes(const WsPlan &plan) {
    size_t off = 0;
    for (auto &p : plan) off += align256(p.second);
    return off;
}

// Points the model's buffers into [base, base + workspace_bytes(plan)).
void carve(const WsPlan &plan, char *base) {
    size_t off = 0;
    for (auto &p : plan) {
        *p.first = base + off;
        off += align256(p.second);
    }
}

int ensure_workspace(fh_model *m, int tokens, int seqs) {
    if (tokens <= m->cap_tokens && seqs <= m->cap_seqs) return FH_OK;
    const int T = std::max(tokens, m->cap_tokens), S = std::max(seqs, m->cap_seqs);
    const auto plan = workspace_plan(m, T, S);
    const size_t bytes = workspace_bytes(plan);
    if (m->ws) {
        HIPCHK(drain(m));
        HIPCHK(hipFree(m->ws));
        m->ws = nullptr;
        m->cap_tokens = m->cap_seqs = 0;
    }
    hipError_t e = hipMalloc(&m->ws, bytes);
    if (e != hipSuccess) return fail(FH_ENOMEM, "workspace hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    m->ws_bytes = bytes;
    carve(plan, (char *)m->ws);
    m->cap_tokens = T;
    m->cap_seqs = S;
    return FH_OK;
}

// ── profiling ──
struct Scope {
    fh_model *m;
    int cls;
    double flops, bytes;
    hipEvent_t a = nullptr, b = nullptr;
    hipStream_t s;
    Scope(fh_model *m_, int c, double f, double by, hipStream_t st) : m(m_), cls(c), flops(f), bytes(by), s(st) {
        if (!m->prof) return;
        a = take();
        b = take();
        hipEventRecord(a, s);
    }
    hipEvent_t take() {
        if (m->event_pool.empty()) {
            hipEvent_t e;
            hipEventCreate(&e);
            return e;
        }
        hipEvent_t e = m->event_pool.back();
        m->event_pool.pop_back();
        return e;
    }
    ~Scope() {
        if (!m->prof) return;
        hipEventRecord(b, s);
        m->pending.push_back({cls, a, b, flops, bytes});
    }
};

void drain_profile(fh_model *m) {
    for (auto &p : m->pending) {
        float ms = 0.f;
        hipEventSynchronize(p.b);
        hipEventElapsedTime(&ms, p.a, p.b);
        m->prof_ms[p.cls] += ms;
        m->prof_flops[p.cls] += p.flops;
        m->prof_bytes[p.cls] += p.bytes;
        m->prof_launches[p.cls] += 1;
        m->event_pool.push_back(p.a);
        m->event_pool.push_back(p.b);
    }
    m->pending.clear();
}

// Cancellation checkpoints observed while the forward executes: at each
// checkpoint an event marks the work enqueued so far, and the host waits
// until the GPU has finished the work before checkpoint k − kPaceAhead
// before it reads the cancel flag and enqueues more.  The GPU keeps up to
// kPaceAhead half-layers queued, so pacing costs it no idle time, and a
// flag raised at any moment during the forward is seen at the next
// checkpoint the GPU reaches (model.go:400, :603 check between layers as
// they run).
constexpr int kPaceAhead = 2;
struct Pacer {
    std::vector<hipEvent_t> ev;  // one per checkpoint passed, in order
    size_t done = 0;             // checkpoints whose preceding work has finished
};

hipEvent_t take_event(fh_model *m) {
    if (m->event_pool.empty()) {
        hipEvent_t e = nullptr;
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return nullptr;
        return e;
    }
    hipEvent_t e = m->event_pool.back();
    m->event_pool.pop_back();
    return e;
}

void release_pacer(fh_model *m, Pacer &p) {
    for (hipEvent_t e : p.ev)
        if (e) m->event_pool.push_back(e);
    p.ev.clear();
    p.done = 0;
}

struct BatchInfo {
    const int32_t *d_ids, *d_offsets;
    int nseq, T, max_len, out_dim;
    float *d_out;
    double sum_l2 = 0.0;  // Σ L_i², for attention FLOP accounting
    const volatile int32_t *cancel = nullptr;
    bool host_checks = false;  // cancellation checkpoints active
    Pacer *pacer = nullptr;    // non-null: pace the enqueue against execution
    int *cp_base = nullptr;    // running checkpoint count across the call's chunks
    // Sequences sorted longest first, the first n_long longer than one key
    // block: attention runs as two launches, [0, n_long) on the multi-block
    // path and [n_long, nseq) (at most max_short tokens) on the one-block
    // path, so each sequence takes its own class's path whatever else is in
    // the batch.  n_long = 0: one launch sized by max_len.
    int n_long = 0, max_short = 0;
};

// Sets n_long/max_short when host offsets show a longest-first batch that
// mixes the two attention classes.
void classify(BatchInfo &b, const int32_t *h_offsets) {
    if (!h_offsets) return;
    int n_long = 0, prev = INT_MAX, max_short = 0;
    for (int i = 0; i < b.nseq; i++) {
        const int L = h_offsets[i + 1] - h_offsets[i];
        if (L > prev) return;  // not longest first: one launch
        prev = L;
        if (L > fh::ATTN_ONE_BLOCK_KEYS) n_long++;
        else max_short = std::max(max_short, L);
    }
    if (n_long > 0 && n_long < b.nseq) {
        b.n_long = n_long;
        b.max_short = max_short;
    }
}

#define LCHK(expr)                                                                         \
    do {                                                                                   \
        hipError_t e_ = (expr);                                                            \
        if (e_ != hipSuccess) return fail(FH_EHIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

int checkpoint(fh_model *m, const BatchInfo &b, int &cp, hipStream_t s) {
    const int idx = (b.cp_base ? *b.cp_base : 0) + cp++;
    if (!b.host_checks) return FH_OK;
    if (Pacer *p = b.pacer) {
        hipEvent_t e = take_event(m);
        if (!e) return fail(FH_EHIP, "hipEventCreate failed");
        p->ev.push_back(e);
        LCHK(hipEventRecord(e, s));
        while (p->ev.size() - p->done > (size_t)kPaceAhead) LCHK(hipEventSynchronize(p->ev[p->done++]));
    }
    const bool hit = (b.cancel && *b.cancel != 0) || (m->cancel_after >= 0 && idx == m->cancel_after);
    if (hit) {
        hipStreamSynchronize(s);
        return fail(FH_ECANCELED, "native: context canceled at checkpoint %d", idx);
    }
    return FH_OK;
}

hipError_t attend(AttnArgs a, const BatchInfo &b, bool out_f32, hipStream_t s) {
    a.seq0 = 0;
    if (b.n_long > 0 && b.n_long < b.nseq) {
        const hipError_t e = fh::attention(a, b.n_long, b.max_len, out_f32, s);
        if (e != hipSuccess) return e;
        a.seq0 = b.n_long;
        return fh::attention(a, b.nseq - b.n_long, b.max_short, out_f32, s);
    }
    return fh::attention(a, b.nseq, b.max_len, out_f32, s);
}

int gemm(fh_model *m, int cls, const DevMat &w, const void *A, int lda, const float *a_scale, int M,
         const float *bias, const float *resid, const f16 *resid_h, int ldr, void *C, int ldc, int act,
         bool out_f32, hipStream_t s) {
    GemmArgs g{};
    g.A = A;
    g.B = w.w;
    g.bias = bias;
    g.resid = resid;
    g.resid_h = resid_h;
    g.a_scale = a_scale;
    g.b_scale = w.scale;
    g.C = C;
    g.M = M;
    g.N = w.n;
    g.K = w.k;
    g.lda = lda;
    g.ldb = w.k;
    g.ldc = ldc;
    g.ldr = ldr;
    const bool i8 = w.scale != nullptr;
    const double flops = 2.0 * M * (double)w.n * w.k;
    const int outn = act == fh::ACT_SWIGLU ? w.n / 2 : w.n;
    const double bytes = (double)M * w.k * (i8 ? 1 : 2) + (double)w.n * w.k * (i8 ? 1 : 2) +
                         (double)M * outn * (out_f32 ? 4 : 2) + (resid ? (double)M * outn * 4 : resid_h ? (double)M * outn * 2 : 0.0);
    Scope sc(m, cls, flops, bytes, s);
    const bool ring = i8 ? w.wr && fh::gemm_ring_worth(M, w.n) && fh::gemm_ring_q8_ok(g, act, out_f32)
                         : use_ring(w, g, act, out_f32, fh::LN_NONE);
    if (ring) g.B = w.wr;
    LCHK(ring ? (i8 ? fh::gemm_ring_q8(g, act, out_f32, s) : fh::gemm_ring(g, act, out_f32, s))
              : i8 ? fh::gemm_i8(g, act, out_f32, s) : fh::gemm_f16(g, act, out_f32, s));
    return FH_OK;
}

// (mean, rstd) of y's rows for the GEMMs that fold LN(y).
int row_stats(fh_model *m, int cls, const f16 *y, int M, f32x2 *st, hipStream_t s) {
    const int H = m->cfg.hidden_size;
    Scope sc(m, cls, 0.0, (double)M * H * 2 + M * 8.0, s);
    LCHK(fh::row_stats(y, M, H, (float)m->cfg.layer_norm_eps, st, s));
    return FH_OK;
}

// Binary16 GEMM whose A operand is the un-normalized input y of a folded
// LayerNorm (LN_IN): C = act(rstd·(y·W'ᵀ − mean·c1) + c2), with y's row
// statistics from row_stats.
int gemm_lnin(fh_model *m, int cls, const DevMat &w, const f16 *y, int M, const float *c1, const float *c2,
              const f32x2 *stats, void *C, int ldc, int act, hipStream_t s) {
    GemmArgs g{};
    g.A = y;
    g.B = w.w;
    g.C = C;
    g.M = M;
    g.N = w.n;
    g.K = w.k;
    g.lda = w.k;
    g.ldb = w.k;
    g.ldc = ldc;
    g.c1 = c1;
    g.c2 = c2;
    g.stats_in = stats;
    const double flops = 2.0 * M * (double)w.n * w.k;
    const int outn = act == fh::ACT_SWIGLU ? w.n / 2 : w.n;
    const double bytes = (double)M * w.k * 2 + (double)w.n * w.k * 2 + (double)M * outn * 2 + M * 8.0;
    Scope sc(m, cls, flops, bytes, s);
    const bool ring = use_ring(w, g, act, false, fh::LN_IN);
    if (ring) g.B = w.wr;
    LCHK(ring ? fh::gemm_ring(g, act, false, s, fh::LN_IN) : fh::gemm_f16(g, act, false, s, fh::LN_IN));
    return FH_OK;
}

// Whether layer L's output projection and feed-forward block run fused for
// M rows: the fragment-ordered copies exist and M is large enough for the
// ring-sized path.
bool use_mlp(const DevLayer &L, int M, int I, bool with_qkv) {
    return L.fc2.wm && L.ffn1.wm && L.out.wm && fh::gemm_ring_worth(M, I) && fh::mlp_ok(M, L.fc2.n, I) &&
           (!with_qkv || fh::mlp_qkv_ok(M));
}

// The rest of the layer after attention in one kernel (fh::mlp with the
// output projection): y = attn·Woᵀ + bo + LNa(ya) (ya's statistics in
// stats_a, γa/βa the previous norm2 or the embedding LayerNorm), then
// out = GELU(LN1(y)·W1ᵀ + b1)·W2ᵀ + b2 + LN1(y), LN1's statistics computed in
// the kernel; stats_out, when set, receives out's statistics for the next
// LayerNorm fold.  out may alias ya and stats_out stats_a (rows belong to
// one block, which reads them before it writes).
int mlp_fused(fh_model *m, const DevLayer &L, const f16 *attn, const f16 *ya, const f32x2 *stats_a,
              const float *ga, const float *ba, int M, f16 *out, f32x2 *stats_out, const DevLayer *next,
              hipStream_t s) {
    const int H = m->cfg.hidden_size, I = m->cfg.intermediate_size;
    MlpArgs g{};
    g.y = nullptr;
    g.stats = nullptr;
    g.attn = attn;
    g.wo = (const f16 *)L.out.wm;
    g.bo = L.out_b;
    g.ya = ya;
    g.stats_a = stats_a;
    g.ga = ga;
    g.ba = ba;
    g.w1 = (const f16 *)L.ffn1.wm;
    g.c1 = L.ffn1_c1;
    g.c2 = L.ffn1_c2;
    g.w2 = (const f16 *)L.fc2.wm;
    g.b2 = L.fc2_b;
    g.ln_g = L.n1w;
    g.ln_b = L.n1b;
    g.out = out;
    g.stats_out = stats_out;
    g.eps = (float)m->cfg.layer_norm_eps;
    g.M = M;
    g.I = I;
    if (next) {  // the next layer's QKV projection of out, into m->qkv
        g.wq = (const f16 *)next->qkv.wm;
        g.c1q = next->qkv_c1;
        g.c2q = next->qkv_c2;
        g.qkv = m->qkv;
    }
    const double flops = 4.0 * M * (double)H * I + 2.0 * M * (double)H * H * (next ? 4 : 1);
    const double bytes = (double)M * H * 2 * 3 + 2.0 * H * I * 2 + 2.0 * H * H * (next ? 4 : 1) + M * 8.0 +
                         (stats_out ? M * 8.0 : 0.0) + (next ? (double)M * 3 * H * 2 : 0.0);
    Scope sc(m, K_MLP, flops, bytes, s);
    LCHK(fh::mlp(g, s));
    return FH_OK;
}

// Binary16 GEMM with the residual LN(yr) rebuilt in the epilogue (RES_LN):
// C = f16(A·Wᵀ + bias + (yr − mean)·rstd·γ + β), yr's statistics from
// row_stats.
int gemm_resln(fh_model *m, int cls, const DevMat &w, const void *A, int M, const float *bias, const f16 *yr,
               const f32x2 *stats, const float *gamma, const float *beta, f16 *C, hipStream_t s,
               const int32_t *res_map = nullptr) {
    GemmArgs g{};
    g.res_map = res_map;
    g.A = A;
    g.B = w.w;
    g.bias = bias;
    g.resid_h = yr;
    g.C = C;
    g.M = M;
    g.N = w.n;
    g.K = w.k;
    g.lda = w.k;
    g.ldb = w.k;
    g.ldc = w.n;
    g.ldr = w.n;
    g.stats_in = stats;
    g.ln_g = gamma;
    g.ln_b = beta;
    const double flops = 2.0 * M * (double)w.n * w.k;
    const double bytes = (double)M * w.k * 2 + (double)w.n * w.k * 2 + (double)M * w.n * 4 + M * 8.0;
    Scope sc(m, cls, flops, bytes, s);
    const bool ring = use_ring(w, g, fh::ACT_NONE, false, fh::RES_LN);
    if (ring) g.B = w.wr;
    LCHK(ring ? fh::gemm_ring(g, fh::ACT_NONE, false, s, fh::RES_LN) : fh::gemm_f16(g, fh::ACT_NONE, false, s, fh::RES_LN));
    return FH_OK;
}

int quant(fh_model *m, const float *x, int M, int K, int ldx, hipStream_t s, int cls = K_QUANT) {
    Scope sc(m, cls, 0.0, (double)M * K * 5, s);
    LCHK(fh::quantize_rows(x, M, K, ldx, m->xq, m->xs, s));
    return FH_OK;
}

// codes: also write the normalized rows' int8 codes and scales to xq/xs
// (the next int8 GEMM's activation quantization, fused).
int layer_norm(fh_model *m, int cls, const float *y32, const f16 *y16, int M, const float *gw, const float *gb,
               float *x32, f16 *x16, hipStream_t s, bool codes = false) {
    const int H = m->cfg.hidden_size;
    Scope sc(m, cls, 0.0, (double)M * H * ((y16 ? 2 : 4) + (x32 ? 4 : 0) + 2 + (codes ? 1 : 0)) + (codes ? M * 4.0 : 0.0),
             s);
    LCHK(fh::layer_norm(y32, y16, M, H, gw, gb, (float)m->cfg.layer_norm_eps, x32, x16, s, codes ? m->xq : nullptr,
                        codes ? m->xs : nullptr));
    return FH_OK;
}

// The pooling stage applies the last LayerNorm (fh::ln_pool / ln_cls_pool)
// from y32 or y16: the un-normalized last hidden state, all T rows (mean) or
// the S compact CLS rows.
int pool_with_ln(fh_model *m, const BatchInfo &b, const float *y32, const f16 *y16, const float *gw, const float *gb,
                 hipStream_t s) {
    const fh_config &c = m->cfg;
    const int H = c.hidden_size, S = b.nseq, od = b.out_dim == 0 ? H : b.out_dim;
    const bool cls = c.pooling == FH_POOL_CLS;
    const double rows = cls ? (double)S : (double)b.T;
    Scope sc(m, K_POOL, 0.0, rows * H * (y32 ? 4 : 2) + (double)S * od * 4, s);
    if (cls)
        LCHK(fh::ln_cls_pool(y32, y16, S, H, gw, gb, (float)c.layer_norm_eps, c.matryoshka_layernorm, od, c.normalize,
                             b.d_out, s));
    else
        LCHK(fh::ln_pool(y32, y16, b.d_offsets, S, b.max_len, H, gw, gb, (float)c.layer_norm_eps,
                         c.matryoshka_layernorm, od, c.normalize, m->pool_part, b.d_out, s));
    return FH_OK;
}

// Forward with every LayerNorm but the last folded into the GEMMs (binary16
// path).  The residual stream is carried un-normalized: yA (x16) is the input
// of the LayerNorm that feeds the attention block (the embedding sum, then
// each layer's y2), yB (y32's storage) the input of norm1.  A small kernel
// records (mean, rstd) per row of y; the QKV and FFN1 GEMMs normalize on the
// fly with them (LN_IN), and the output projection and FC2 rebuild their
// residual LN(y) from the same statistics (RES_LN) and write the next
// un-normalized y.  Only the last layer's norm2 runs as a kernel, producing
// the f32 rows pooling reads.
int run_forward_fold(fh_model *m, const BatchInfo &b, hipStream_t s) {
    const fh_config &c = m->cfg;
    const int H = c.hidden_size, I = c.intermediate_size, T = b.T, S = b.nseq;
    const bool cls = c.pooling == FH_POOL_CLS, swiglu = c.activation == FH_ACT_SWIGLU;
    f16 *const yB = (f16 *)m->y32;
    int cp = 0, rc;
    {
        Scope sc(m, K_EMBED, 0.0, (double)T * H * (4 + (m->pos ? 4 : 0) + 2) + T * 4.0, s);
        // The first layer's QKV fold needs the sum's row statistics: written
        // here with it where the kernel covers the width.
        LCHK(fh::embed_ln(b.d_ids, b.d_offsets, S, b.max_len, m->word, m->type0, m->pos, nullptr, nullptr,
                          (float)c.layer_norm_eps, H, nullptr, m->x16, s, nullptr, nullptr, 0,
                          m->embed_stats ? m->sA : nullptr));
    }
    // sA already holds yA's statistics (written by the embedding kernel or
    // the previous fused kernel)
    bool sa_ready = m->embed_stats;
    bool qkv_ready = false;  // qkv already holds this layer's projection (ditto)
    for (int li = 0; li < c.num_layers; li++) {
        const DevLayer &L = m->layers[(size_t)li];
        if ((rc = checkpoint(m, b, cp, s))) return rc;
        const bool last = li == c.num_layers - 1, last_cls = cls && last;
        const float *gA = li ? m->layers[(size_t)li - 1].n2w : m->emb_w;
        const float *bA = li ? m->layers[(size_t)li - 1].n2b : m->emb_b;

        // qkv = LN(yA)·Wqkvᵀ + b  (model.go:555)
        if (!qkv_ready &&
            ((!sa_ready && (rc = row_stats(m, K_STATS, m->x16, T, m->sA, s))) ||
             (rc = gemm_lnin(m, K_GEMM_QKV, L.qkv, m->x16, T, L.qkv_c1, L.qkv_c2, m->sA, m->qkv, 3 * H, fh::ACT_NONE,
                             s))))
            return rc;

        // attention (model.go:557-593, 646-701)
        AttnArgs a{};
        a.qkv = m->qkv;
        a.offsets = b.d_offsets;
        a.rope_cos = m->rope_cos;
        a.rope_sin = m->rope_sin;
        a.out = last_cls ? m->attnc : m->attn;
        a.H = H;
        a.d = m->hd;
        a.ldo = H;
        a.q_limit = last_cls ? 1 : INT_MAX;
        a.compact = last_cls ? 1 : 0;
        a.scale_log2e = (float)(1.0 / std::sqrt((double)m->hd)) * 1.4426950408889634f;
        {
            const double nq_l = last_cls ? (double)T : b.sum_l2;
            Scope sc(m, last_cls ? K_CLS_TAIL : K_ATTN, 4.0 * nq_l * H, (double)T * 3 * H * 2 + (last_cls ? S : T) * (double)H * 2,
                     s);
            if (rope_pre(m)) {  // as in run_forward
                LCHK(fh::rope_qk(m->qkv, b.d_offsets, b.nseq, b.max_len, H, m->hd, m->rope_cos, m->rope_sin, s));
                a.rope_cos = a.rope_sin = nullptr;
            }
            LCHK(attend(a, b, false, s));
        }

        const int M = last_cls ? S : T;
        f16 *yA = last_cls ? m->xc16 : m->x16, *yBo = last_cls ? m->yBc : yB;
        f32x2 *sA = last_cls ? m->sAc : m->sA, *sB = last_cls ? m->sBc : m->sB;
        const DevLayer *next = last ? nullptr : &m->layers[(size_t)li + 1];
        if (next && !next->qkv.wm) next = nullptr;
        const bool fused = use_mlp(L, M, I, next != nullptr);
        // The CLS rows' residual: gathered into compact rows, except where
        // the output projection runs on the tiled GEMM, which reads the CLS
        // rows of the full-token stream through a row map (the offsets).
        const bool res_map = last_cls && !fused && !fh::gemm_ring_worth(M, L.out.n);
        if (last_cls && !res_map) {
            Scope sc(m, K_CLS_TAIL, 0.0, (double)S * (H * 4 + 16), s);
            LCHK(fh::gather_rows(nullptr, m->x16, m->sA, b.d_offsets, S, H, nullptr, m->xc16, m->sAc, s));
        }
        // The CLS layer's compact (M = nseq) GEMMs count in the GEMM
        // classes; its attention, gather and statistics in cls_last_layer.
        const int kOut = K_GEMM_OUT, kFfn1 = K_GEMM_FFN1, kFc2 = K_GEMM_FC2;

        sa_ready = qkv_ready = false;
        if (fused) {
            // yB = attn·Woᵀ + b + LN(yA), then the feed-forward block, in one
            // kernel: yB stays on-chip, its statistics are computed there,
            // and (unless this is the last layer) so are the new yA's for the
            // next layer's QKV fold.  The checkpoint between the two
            // (model.go:603) is taken before the launch.
            // The next layer's QKV projection (over all T rows, also for the
            // CLS-pooled last layer) runs at the end of the same kernel.
            if ((rc = checkpoint(m, b, cp, s)) ||
                (rc = mlp_fused(m, L, (const f16 *)(last_cls ? m->attnc : m->attn), yA, sA, gA, bA, M, yA,
                                last ? nullptr : m->sA, next, s)))
                return rc;
            sa_ready = !last;
            qkv_ready = next != nullptr;
            continue;
        }
        // yB = attn·Woᵀ + b + LN(yA)  (model.go:596-599)
        if ((rc = gemm_resln(m, kOut, L.out, last_cls ? m->attnc : m->attn, M, L.out_b, res_map ? m->x16 : yA,
                             res_map ? m->sA : sA, gA, bA, yBo, s, res_map ? b.d_offsets : nullptr)))
            return rc;
        if ((rc = checkpoint(m, b, cp, s))) return rc;

        // h = act(LN1(yB)·W1ᵀ + b1); yA = h·W2ᵀ + b2 + LN1(yB)  (model.go:607-633)
        if ((rc = row_stats(m, last_cls ? K_CLS_TAIL : K_STATS, yBo, M, sB, s)) ||
            (rc = gemm_lnin(m, kFfn1, L.ffn1, yBo, M, L.ffn1_c1, L.ffn1_c2, sB, m->hbuf, I,
                            swiglu ? fh::ACT_SWIGLU : fh::ACT_GELU, s)))
            return rc;
        if ((rc = gemm_resln(m, kFc2, L.fc2, m->hbuf, M, L.fc2_b, yBo, sB, L.n1w, L.n1b, yA, s))) return rc;
    }
    // The last norm2, to f32 rows for pooling (or inside the mean pooling).
    const DevLayer &Lz = m->layers.back();
    if (m->ln_pool) return pool_with_ln(m, b, nullptr, cls ? m->xc16 : m->x16, Lz.n2w, Lz.n2b, s);
    if ((rc = layer_norm(m, K_LN, nullptr, cls ? m->xc16 : m->x16, cls ? S : T, Lz.n2w, Lz.n2b, cls ? m->xc32 : m->x32,
                         nullptr, s)))
        return rc;
    {
        const int od = b.out_dim == 0 ? H : b.out_dim;
        Scope sc(m, K_POOL, 0.0, (cls ? (double)S * H * 4 : (double)T * H * 4) + (double)S * od * 4, s);
        LCHK(fh::pool(cls ? m->xc32 : m->x32, b.d_offsets, S, b.max_len, H, cls ? 1 : 0, cls ? 0 : 1,
                      c.matryoshka_layernorm, od, c.normalize, m->pool_part, b.d_out, s));
    }
    return FH_OK;
}

int run_forward(fh_model *m, const BatchInfo &b, hipStream_t s) {
    if (m->lnfold) return run_forward_fold(m, b, s);
    const fh_config &c = m->cfg;
    const int H = c.hidden_size, I = c.intermediate_size, T = b.T, S = b.nseq;
    const bool q8 = c.q8 != 0, cls = c.pooling == FH_POOL_CLS, swiglu = c.activation == FH_ACT_SWIGLU;
    const float eps = (float)c.layer_norm_eps;
    // Residual stream: binary16 between layers, except on the Q8 path, whose
    // activation quantizer reads the f32 stream like quant.go:104-110.  On
    // the binary16 path the projection GEMMs add bias and residual in f32 and
    // round once to binary16 (y16, aliasing y32's storage) for the LN; the
    // last layer's LN always writes f32 for pooling.
    const bool f32res = q8;
    f16 *const y16 = (f16 *)m->y32;
    int cp = 0, rc;

    {
        Scope sc(m, K_EMBED, 0.0, (double)T * H * (4 + (m->pos ? 4 : 0) + (f32res ? 6 : 2) + (q8 ? 1 : 0)) + T * 4.0,
                 s);
        // Q8: with the first layer's activation codes
        LCHK(fh::embed_ln(b.d_ids, b.d_offsets, S, b.max_len, m->word, m->type0, m->pos, m->emb_w, m->emb_b,
                          eps, H, f32res ? m->x32 : nullptr, m->x16, s, q8 ? m->xq : nullptr, q8 ? m->xs : nullptr,
                          T));
    }
    for (int li = 0; li < c.num_layers; li++) {
        const DevLayer &L = m->layers[(size_t)li];
        if ((rc = checkpoint(m, b, cp, s))) return rc;
        const bool last = li == c.num_layers - 1, last_cls = cls && last;

        // qkv = x·Wqkvᵀ + b  (model.go:555); Q8: x's codes come from the
        // LayerNorm that produced x (the embedding LN or the previous norm2)
        if (q8) {
            rc = gemm(m, K_GEMM_QKV, L.qkv, m->xq, H, m->xs, T, L.qkv_b, nullptr, nullptr, 0, m->qkv, 3 * H,
                      fh::ACT_NONE, false, s);
        } else {
            rc = gemm(m, K_GEMM_QKV, L.qkv, m->x16, H, nullptr, T, L.qkv_b, nullptr, nullptr, 0, m->qkv, 3 * H,
                      fh::ACT_NONE, false, s);
        }
        if (rc) return rc;

        // attention (model.go:557-593, 646-701)
        AttnArgs a{};
        a.qkv = m->qkv;
        a.offsets = b.d_offsets;
        a.rope_cos = m->rope_cos;
        a.rope_sin = m->rope_sin;
        a.out = last_cls ? m->attnc : m->attn;
        a.H = H;
        a.d = m->hd;
        a.ldo = H;
        a.q_limit = last_cls ? 1 : INT_MAX;
        a.compact = last_cls ? 1 : 0;
        a.scale_log2e = (float)(1.0 / std::sqrt((double)m->hd)) * 1.4426950408889634f;
        {
            const double nq_l = last_cls ? (double)T : b.sum_l2;  // Σ nq·L
            Scope sc(m, last_cls ? K_CLS_TAIL : K_ATTN, 4.0 * nq_l * H, (double)T * 3 * H * 2 + (last_cls ? S : T) * (double)H * (q8 ? 4 : 2),
                     s);
            // RoPE: Q and K rotated once per token in place, then attention
            // without it (the same bits as rotating inside attention).
            if (rope_pre(m)) {
                LCHK(fh::rope_qk(m->qkv, b.d_offsets, b.nseq, b.max_len, H, m->hd, m->rope_cos, m->rope_sin, s));
                a.rope_cos = a.rope_sin = nullptr;
            }
            LCHK(attend(a, b, q8, s));
        }

        const int M = last_cls ? S : T;
        float *xo32 = last_cls ? m->xc32 : m->x32;
        f16 *xo16 = last_cls ? m->xc16 : m->x16;
        const void *attn_in = last_cls ? m->attnc : m->attn;
        if (last_cls) {
            Scope sc(m, K_CLS_TAIL, 0.0, (double)S * H * (f32res ? 8 : 4), s);
            LCHK(fh::gather_rows(f32res ? m->x32 : nullptr, f32res ? nullptr : m->x16, nullptr, b.d_offsets, S, H,
                                 f32res ? m->xc32 : nullptr, f32res ? nullptr : m->xc16, nullptr, s));
        }
        const int kOut = K_GEMM_OUT, kLn = last_cls ? K_CLS_TAIL : K_LN;
        const int kFfn1 = K_GEMM_FFN1, kFc2 = K_GEMM_FC2;
        const int kQuant = last_cls ? K_CLS_TAIL : K_QUANT;
        const float *r32 = f32res ? xo32 : nullptr;
        const f16 *r16 = f32res ? nullptr : xo16;

        // out projection + bias + residual, norm1 (model.go:596-599)
        if (q8) {
            if ((rc = quant(m, (const float *)attn_in, M, H, H, s, kQuant))) return rc;
            rc = gemm(m, kOut, L.out, m->xq, H, m->xs, M, L.out_b, r32, r16, H, m->y32, H, fh::ACT_NONE,
                      true, s);
        } else {
            rc = gemm(m, kOut, L.out, attn_in, H, nullptr, M, L.out_b, r32, r16, H, y16, H, fh::ACT_NONE,
                      false, s);
        }
        if (rc) return rc;
        if ((rc = layer_norm(m, kLn, f32res ? m->y32 : nullptr, f32res ? nullptr : y16, M, L.n1w, L.n1b,
                             f32res ? xo32 : nullptr, xo16, s, q8)))
            return rc;

        if ((rc = checkpoint(m, b, cp, s))) return rc;

        // FFN (model.go:607-633)
        const int act = swiglu ? fh::ACT_SWIGLU : fh::ACT_GELU;
        if (q8) {  // x1's codes from norm1 above
            if ((rc = gemm(m, kFfn1, L.ffn1, m->xq, H, m->xs, M, L.ffn1_b, nullptr, nullptr, 0, m->hbuf, I,
                           act, true, s)))
                return rc;
            if ((rc = quant(m, (const float *)m->hbuf, M, I, I, s, kQuant))) return rc;
            rc = gemm(m, kFc2, L.fc2, m->xq, I, m->xs, M, L.fc2_b, r32, r16, H, m->y32, H, fh::ACT_NONE, true,
                      s);
        } else {
            if ((rc = gemm(m, kFfn1, L.ffn1, xo16, H, nullptr, M, L.ffn1_b, nullptr, nullptr, 0, m->hbuf, I,
                           act, false, s)))
                return rc;
            rc = gemm(m, kFc2, L.fc2, m->hbuf, I, nullptr, M, L.fc2_b, r32, r16, H, y16, H, fh::ACT_NONE,
                      false, s);
        }
        if (rc) return rc;
        // norm2; Q8: with the next layer's QKV activation codes.  The last
        // one is left to the mean pooling when that fuses it.
        if (last && m->ln_pool)
            return pool_with_ln(m, b, f32res ? m->y32 : nullptr, f32res ? nullptr : y16, L.n2w, L.n2b, s);
        if ((rc = layer_norm(m, kLn, f32res ? m->y32 : nullptr, f32res ? nullptr : y16, M, L.n2w, L.n2b,
                             (f32res || last) ? xo32 : nullptr, xo16, s, q8 && !last)))
            return rc;
    }

    // pooling → Matryoshka → L2 (model.go:417-453)
    {
        const int od = b.out_dim == 0 ? H : b.out_dim;
        Scope sc(m, K_POOL, 0.0, (cls ? (double)S * H * 4 : (double)T * H * 4) + (double)S * od * 4, s);
        LCHK(fh::pool(cls ? m->xc32 : m->x32, b.d_offsets, S, b.max_len, H, cls ? 1 : 0, cls ? 0 : 1,
                      c.matryoshka_layernorm, od, c.normalize, m->pool_part, b.d_out, s));
    }
    return FH_OK;
}

}  // namespace

// ───────────────────────────── C ABI ─────────────────────────────

extern "C" void fh_model_destroy(fh_model *m) {
    if (!m) return;
    hipSetDevice(m->device);
    if (m->stream) hipStreamSynchronize(m->stream);
    for (auto &p : m->pending) {
        hipEventDestroy(p.a);
        hipEventDestroy(p.b);
    }
    for (auto e : m->event_pool) hipEventDestroy(e);
    if (m->done_ev) {
        if (m->done_stream) hipEventSynchronize(m->done_ev);
        hipEventDestroy(m->done_ev);
    }
    for (void *p : m->allocs) hipFree(p);
    if (m->ws) hipFree(m->ws);
    if (m->io) hipFree(m->io);
    if (m->pin) hipHostFree(m->pin);
    if (m->stream) hipStreamDestroy(m->stream);
    delete m;
}

extern "C" int fh_model_create(const fh_config *cfg, const fh_tensor *tensors, int32_t n_tensors, int32_t device,
                               fh_model **out) {
    if (!cfg || !out || (n_tensors > 0 && !tensors)) return fail(FH_EINVAL, "fh_model_create: null argument");
    *out = nullptr;
    const fh_config &c = *cfg;
    if (c.hidden_size <= 0 || c.num_layers <= 0 || c.num_heads <= 0 || c.intermediate_size <= 0 ||
        c.vocab_size <= 0 || c.max_seq_len <= 2 || c.layer_norm_eps <= 0)
        return fail(FH_EINVAL, "pack: non-positive architecture dimension");
    if (c.hidden_size % c.num_heads) return fail(FH_EINVAL, "pack: hidden_size not divisible by num_heads");
    const int H = c.hidden_size, I = c.intermediate_size, hd = H / c.num_heads;
    // Shape limits of this build's kernels (16-byte vector tiles, LN row in registers).
    if (H > 1024 || H % 8 || I % 16 || hd % 8 || hd > 128)
        return fail(FH_EINVAL, "pack: shape H=%d I=%d head_dim=%d outside this build's kernel limits "
                               "(H ≤ 1024, H%%8 = 0, I%%16 = 0, head_dim%%8 = 0, head_dim ≤ 128)", H, I, hd);
    if (c.position_encoding == FH_POS_ROPE && c.rope_theta <= 0)
        return fail(FH_EINVAL, "pack: rope position encoding requires rope_theta > 0");

    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return fail(FH_ENODEV, "no HIP device visible");
    if (device < 0 || device >= ndev) return fail(FH_ENODEV, "device %d outside [0,%d)", device, ndev);
    hipDeviceProp_t prop;
    HIPCHK(hipGetDeviceProperties(&prop, device));
    if (!strstr(prop.gcnArchName, "gfx950"))
        return fail(FH_ENODEV, "device %d is %s; this library is built for gfx950 only", device, prop.gcnArchName);
    HIPCHK(hipSetDevice(device));
    if (int rs = init_scratch(device)) return rs;

    fh_model *m = new fh_model();
    m->cfg = c;
    m->device = device;
    m->hd = hd;
    m->eff_max = eff_max_len(c);
    if (const char *ct = getenv("FUTON_CHUNK_TOKENS")) {
        const long v = strtol(ct, nullptr, 10);
        if (v > 0 && v < INT_MAX) m->chunk_tokens = (int)v;
    }
    m->chunk_tokens = std::max(m->chunk_tokens, m->eff_max);  // a chunk always holds the longest sequence
    if (const char *sc = getenv("FUTON_SCHEDULE")) m->schedule = sc[0] != '0';
    int rc = FH_OK;
    auto bail = [&](int code) {
        fh_model_destroy(m);
        return code;
    };
    if (hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess)
        return bail(fail(FH_EHIP, "hipStreamCreate failed"));
    if (hipEventCreateWithFlags(&m->done_ev, hipEventDisableTiming) != hipSuccess)
        return bail(fail(FH_EHIP, "hipEventCreate failed"));

    Loader ld{m, tensors, n_tensors, std::vector<bool>((size_t)n_tensors, false)};
    if ((rc = ld.mat_f32("embeddings.word", c.vocab_size, H, &m->word))) return bail(rc);
    if (c.position_encoding == FH_POS_ABSOLUTE &&
        (rc = ld.mat_f32("embeddings.position", c.max_seq_len, H, &m->pos)))
        return bail(rc);
    if (c.type_vocab_size > 0) {
        // Only token type 0 is ever added (model.go:388-390); the table is validated whole.
        TensorView tv;
        if ((rc = ld.need("embeddings.token_type", {c.type_vocab_size, H}, tv))) return bail(rc);
        std::vector<float> t;
        tv.to_f32(t);
        if ((rc = upload(m, &m->type0, t.data(), (size_t)H * 4))) return bail(rc);
    }
    if ((rc = ld.vec_f32("embeddings.norm.weight", H, &m->emb_w))) return bail(rc);
    if ((rc = ld.vec_f32("embeddings.norm.bias", H, &m->emb_b))) return bail(rc);

    const bool swiglu = c.activation == FH_ACT_SWIGLU, q8 = c.q8 != 0;
    // Fold the LayerNorms into the GEMMs on the binary16 path for the row
    // widths the un-normalized embedding kernel covers; FUTON_LN_FOLD=0 keeps
    // the separate LayerNorm kernels (diagnostics).
    const char *fold_env = getenv("FUTON_LN_FOLD");
    m->lnfold = !q8 && H % 64 == 0 && (H / 64 == 4 || H / 64 == 6 || H / 64 == 8 || H / 64 == 12 || H / 64 == 16) &&
                !(fold_env && fold_env[0] == '0');
    // The folded binary16 projections run on the persistent ring GEMM when
    // their shape fits it (N % 128, K % 64; the SwiGLU pair too);
    // FUTON_GEMM_RING=0 keeps them on the tiled GEMM (diagnostics).
    // The int8 projections of the Q8 path run on the ring GEMM's int8 form
    // (N % 128, K % 128).
    const char *ring_env = getenv("FUTON_GEMM_RING");
    const bool ring_env_on = !(ring_env && ring_env[0] == '0');
    const bool ring_on = m->lnfold && ring_env_on;
    auto ring_fits = [&](int n, int k) {
        return q8 ? ring_env_on && n % 128 == 0 && k % 128 == 0 : ring_on && n % 128 == 0 && k % 64 == 0;
    };
    // The feed-forward block runs fused (fh::mlp) for hidden width 384 with
    // GELU; FUTON_MLP=0 keeps the two ring GEMMs (diagnostics).
    const char *mlp_env = getenv("FUTON_MLP");
    const bool mlp_on = ring_on && !swiglu && !(mlp_env && mlp_env[0] == '0') && fh::mlp_ok(1, H, I) &&
                        ring_fits(I, H);
    std::vector<float> gA, bA, g1, b1, bias, c1, c2;
    if (m->lnfold && ((rc = ld.vec_host("embeddings.norm.weight", H, gA)) ||
                      (rc = ld.vec_host("embeddings.norm.bias", H, bA))))
        return bail(rc);
    m->layers.resize((size_t)c.num_layers);
    std::vector<float> w, g, packed;
    for (int li = 0; li < c.num_layers; li++) {
        DevLayer &L = m->layers[(size_t)li];
        auto nm = [&](const char *s) { return "layers." + std::to_string(li) + "." + s; };
        if ((rc = ld.mat_host(nm("attn.qkv.weight"), 3 * H, H, w))) return bail(rc);
        if (m->lnfold) {
            if ((rc = ld.vec_host(nm("attn.qkv.bias"), 3 * H, bias, true))) return bail(rc);
            fold_ln(w, 3 * H, H, gA, bA, bias, c1, c2);
            if ((rc = upload(m, &L.qkv_c1, c1.data(), c1.size() * 4)) ||
                (rc = upload(m, &L.qkv_c2, c2.data(), c2.size() * 4)))
                return bail(rc);
        }
        if ((rc = upload_mat(m, L.qkv, w, 3 * H, H, q8, ring_fits(3 * H, H), mlp_on ? 2 : 0))) return bail(rc);
        if ((rc = ld.vec_f32(nm("attn.qkv.bias"), 3 * H, &L.qkv_b, true))) return bail(rc);
        if ((rc = ld.mat_host(nm("attn.out.weight"), H, H, w)) ||
            (rc = upload_mat(m, L.out, w, H, H, q8, ring_fits(H, H), mlp_on ? 2 : 0)))
            return bail(rc);
        if ((rc = ld.vec_f32(nm("attn.out.bias"), H, &L.out_b, true))) return bail(rc);
        if ((rc = ld.vec_f32(nm("norm1.weight"), H, &L.n1w)) || (rc = ld.vec_f32(nm("norm1.bias"), H, &L.n1b)))
            return bail(rc);
        if (m->lnfold &&
            ((rc = ld.vec_host(nm("norm1.weight"), H, g1)) || (rc = ld.vec_host(nm("norm1.bias"), H, b1))))
            return bail(rc);
        if ((rc = ld.mat_host(nm("mlp.fc1.weight"), I, H, w))) return bail(rc);
        if (swiglu) {
            if ((rc = ld.mat_host(nm("mlp.gate.weight"), I, H, g))) return bail(rc);
            interleave16(w, g, I, H, packed);
            // biases follow the same interleave (absent biases stay absent)
            TensorView tb1, tb2;
            bool p1 = false, p2 = false;
            if ((rc = ld.need(nm("mlp.fc1.bias"), {I}, tb1, true, &p1)) ||
                (rc = ld.need(nm("mlp.gate.bias"), {I}, tb2, true, &p2)))
                return bail(rc);
            std::vector<float> bp;
            if (p1 || p2) {
                std::vector<float> bu((size_t)I, 0.f), bg((size_t)I, 0.f);
                bp.resize((size_t)2 * I);
                if (p1) tb1.to_f32(bu);
                if (p2) tb2.to_f32(bg);
                for (int r = 0; r < 2 * I; r++) {
                    const int blk = r / 32, ww = r % 32;
                    bp[(size_t)r] = ww < 16 ? bu[(size_t)(16 * blk + ww)] : bg[(size_t)(16 * blk + ww - 16)];
                }
                if ((rc = upload(m, &L.ffn1_b, bp.data(), bp.size() * 4))) return bail(rc);
            }
            if (m->lnfold) {
                fold_ln(packed, 2 * I, H, g1, b1, bp, c1, c2);
                if ((rc = upload(m, &L.ffn1_c1, c1.data(), c1.size() * 4)) ||
                    (rc = upload(m, &L.ffn1_c2, c2.data(), c2.size() * 4)))
                    return bail(rc);
            }
            if ((rc = upload_mat(m, L.ffn1, packed, 2 * I, H, q8, ring_fits(2 * I, H)))) return bail(rc);
        } else {
            if (m->lnfold) {
                if ((rc = ld.vec_host(nm("mlp.fc1.bias"), I, bias, true))) return bail(rc);
                fold_ln(w, I, H, g1, b1, bias, c1, c2);
                if ((rc = upload(m, &L.ffn1_c1, c1.data(), c1.size() * 4)) ||
                    (rc = upload(m, &L.ffn1_c2, c2.data(), c2.size() * 4)))
                    return bail(rc);
            }
            if ((rc = upload_mat(m, L.ffn1, w, I, H, q8, ring_fits(I, H), mlp_on ? 1 : 0))) return bail(rc);
            if ((rc = ld.vec_f32(nm("mlp.fc1.bias"), I, &L.ffn1_b, true))) return bail(rc);
        }
        if ((rc = ld.mat_host(nm("mlp.fc2.weight"), H, I, w)) ||
            (rc = upload_mat(m, L.fc2, w, H, I, q8, ring_fits(H, I), mlp_on ? 2 : 0)))
            return bail(rc);
        if ((rc = ld.vec_f32(nm("mlp.fc2.bias"), H, &L.fc2_b, true))) return bail(rc);
        if ((rc = ld.vec_f32(nm("norm2.weight"), H, &L.n2w)) || (rc = ld.vec_f32(nm("norm2.bias"), H, &L.n2b)))
            return bail(rc);
        if (m->lnfold &&
            ((rc = ld.vec_host(nm("norm2.weight"), H, gA)) || (rc = ld.vec_host(nm("norm2.bias"), H, bA))))
            return bail(rc);
    }
    for (int i = 0; i < n_tensors; i++) {
        if (!ld.used[(size_t)i])
            return bail(fail(FH_EINVAL, "pack: unexpected tensor \"%s\" (pack/config mismatch)",
                             tensors[i].name ? tensors[i].name : "(null)"));
    }
    if (c.position_encoding == FH_POS_ROPE) {
        // native/model.go:306-318: float64 angles, float32 tables, effective max positions.
        const int half = hd / 2, n = m->eff_max;
        std::vector<float> cs((size_t)n * half), sn((size_t)n * half);
        for (int t = 0; t < n; t++)
            for (int i = 0; i < half; i++) {
                const double freq = 1.0 / std::pow(c.rope_theta, (double)(2 * i) / (double)hd);
                const double ang = (double)t * freq;
                cs[(size_t)t * half + i] = (float)std::cos(ang);
                sn[(size_t)t * half + i] = (float)std::sin(ang);
            }
        if ((rc = upload(m, &m->rope_cos, cs.data(), cs.size() * 4)) ||
            (rc = upload(m, &m->rope_sin, sn.data(), sn.size() * 4)))
            return bail(rc);
        const char *rq = getenv("FUTON_ROPE_QK");
        m->rope_pre = !(rq && rq[0] == '0') && fh::rope_qk_ok(H, hd);
    }
    {
        const char *lp = getenv("FUTON_LN_POOL");
        m->ln_pool = !(lp && lp[0] == '0') && fh::ln_pool_ok(H);
        const char *es = getenv("FUTON_EMBED_STATS");
        m->embed_stats = !(es && es[0] == '0') && fh::embed_stats_ok(H);
    }
    *out = m;
    return FH_OK;
}

extern "C" int64_t fh_model_device_bytes(const fh_model *m) {
    return m ? m->weight_bytes + (int64_t)m->ws_bytes : 0;
}

extern "C" int fh_checkpoints_per_call(const fh_model *m) { return m ? 2 * m->cfg.num_layers : 0; }

extern "C" int fh_debug_cancel_after(fh_model *m, int32_t n) {
    if (!m) return fail(FH_EINVAL, "null model");
    std::lock_guard<std::mutex> lk(m->mu);
    m->cancel_after = n;
    return FH_OK;
}

extern "C" int fh_encode(fh_model *m, const int32_t *ids, const int32_t *seq_offsets, int32_t nseq,
                         int32_t out_dim, float *out, const volatile int32_t *cancel) {
    if (!m) return fail(FH_EINVAL, "native: null model");
    if (nseq < 0) return fail(FH_EINVAL, "native: negative batch size");
    if (nseq == 0) return FH_OK;
    if (!ids || !seq_offsets || !out) return fail(FH_EINVAL, "native: null buffer");
    const fh_config &c = m->cfg;
    if (seq_offsets[0] != 0) return fail(FH_EINVAL, "native: seq_offsets[0] must be 0");
    // Per-sequence validation in the reference's order (model.go:348-365).
    for (int i = 0; i < nseq; i++) {
        const int L = seq_offsets[i + 1] - seq_offsets[i];
        if (L <= 0) return fail(FH_EINVAL, "native: batch item %d: native: empty token sequence", i);
        if (L > m->eff_max)
            return fail(FH_ETOOLONG,
                        "native: batch item %d: native: sequence length %d exceeds effective max_seq_len %d "
                        "(declared %d, trained %d)",
                        i, L, m->eff_max, c.max_seq_len, c.max_trained_positions);
        if (out_dim < 0 || out_dim > c.hidden_size)
            return fail(FH_EINVAL, "native: batch item %d: native: requested dim %d outside [1,%d]", i, out_dim,
                        c.hidden_size);
        if (out_dim != 0 && out_dim != c.hidden_size && !c.matryoshka)
            return fail(FH_EINVAL, "native: batch item %d: native: pack does not support matryoshka truncation to %d",
                        i, out_dim);
        for (int t = seq_offsets[i]; t < seq_offsets[i + 1]; t++) {
            if (ids[t] < 0 || ids[t] >= c.vocab_size)
                return fail(FH_EINVAL, "native: batch item %d: native: token id %d outside vocab of %d", i, ids[t],
                            c.vocab_size);
        }
    }
    const int T = seq_offsets[nseq];
    const int od = out_dim == 0 ? c.hidden_size : out_dim;

    // Schedule (the batch counterpart of the reference's longest-first
    // dispatch, provider.go:183-246): sequences sorted longest first and cut
    // into chunks of at most chunk_tokens tokens, each one packed forward.
    // Inside a chunk the sequences longer than one key block
    // (fh::ATTN_ONE_BLOCK_KEYS) form a prefix, and attention runs once over
    // that prefix and once over the rest, so a long sequence does not move
    // the short ones onto the multi-block path while the GEMMs still see the
    // whole chunk.  A sequence's vector (fixed reduction orders, kernels
    // chosen only by its own class) is then the same bits in any batch.
    std::vector<int> ord((size_t)nseq);
    for (int i = 0; i < nseq; i++) ord[(size_t)i] = i;
    auto len = [&](int i) { return seq_offsets[i + 1] - seq_offsets[i]; };
    if (m->schedule) std::stable_sort(ord.begin(), ord.end(), [&](int a, int b) { return len(a) > len(b); });
    struct Chunk {
        int s0, ns, t0, nt, max_len;
        double sum_l2;
        int n_long, max_short;  // sequences past one key block (a prefix: longest first), longest of the rest
    };
    std::vector<Chunk> chunks;
    int max_nt = 0, max_ns = 0;
    {
        int t = 0;
        for (int j = 0; j < nseq; j++) {
            const int L = len(ord[(size_t)j]);
            const bool one = L <= fh::ATTN_ONE_BLOCK_KEYS;
            if (chunks.empty() || chunks.back().nt + L > m->chunk_tokens) chunks.push_back({j, 0, t, 0, L, 0.0, 0, 0});
            Chunk &k = chunks.back();
            k.max_len = std::max(k.max_len, L);
            if (m->schedule && !one) k.n_long++;
            if (one) k.max_short = std::max(k.max_short, L);
            k.ns++;
            k.nt += L;
            k.sum_l2 += (double)L * L;
            t += L;
            max_nt = std::max(max_nt, k.nt);
            max_ns = std::max(max_ns, k.ns);
        }
    }
    const int nch = (int)chunks.size();
    // I/O layout: ids in schedule order | chunk-local offsets (ns + 1 per
    // chunk) | vectors in schedule order.
    const size_t off_ids = 0, off_offs = align256((size_t)T * 4);
    const size_t off_out = off_offs + align256((size_t)(nseq + nch) * 4);
    const size_t io_need = off_out + (size_t)nseq * od * 4;

    std::lock_guard<std::mutex> lk(m->mu);
    HIPCHK(hipSetDevice(m->device));
    int rc = ensure_workspace(m, max_nt, max_ns);
    if (rc || (rc = ensure_io(m, io_need))) return rc;
    // The staging buffer is free: every earlier forward that read it has
    // finished (fh_encode waits for its own before returning).
    int32_t *p_ids = (int32_t *)((char *)m->pin + off_ids), *p_off = (int32_t *)((char *)m->pin + off_offs);
    const float *p_out = (const float *)((char *)m->pin + off_out);
    {
        int32_t *pi = p_ids, *po = p_off;
        for (const Chunk &k : chunks) {
            int32_t acc = 0;
            *po++ = 0;
            for (int j = k.s0; j < k.s0 + k.ns; j++) {
                const int i = ord[(size_t)j], L = len(i);
                memcpy(pi, ids + seq_offsets[i], (size_t)L * 4);
                pi += L;
                acc += L;
                *po++ = acc;
            }
        }
    }
    hipStream_t s = m->stream;
    if ((rc = begin_on(m, s))) return rc;
    char *io = (char *)m->io;
    HIPCHK(hipMemcpyAsync(io, m->pin, off_out, hipMemcpyHostToDevice, s));
    // Pace the enqueue against execution only when something can cancel.
    Pacer pacer;
    const bool pace = cancel != nullptr || m->cancel_after >= 0;
    int cp_base = 0;
    for (int ci = 0; ci < nch && rc == FH_OK; ci++) {
        const Chunk &k = chunks[(size_t)ci];
        BatchInfo b{(const int32_t *)(io + off_ids) + k.t0, (const int32_t *)(io + off_offs) + k.s0 + ci, k.ns, k.nt,
                    k.max_len, out_dim, (float *)(io + off_out) + (size_t)k.s0 * od};
        b.sum_l2 = k.sum_l2;
        if (k.n_long > 0 && k.n_long < k.ns) {
            b.n_long = k.n_long;
            b.max_short = k.max_short;
        }
        b.cancel = cancel;
        b.host_checks = true;
        b.pacer = pace ? &pacer : nullptr;
        b.cp_base = &cp_base;
        rc = run_forward(m, b, s);
        cp_base += 2 * c.num_layers;
    }
    if (rc == FH_OK) {
        const hipError_t e = hipMemcpyAsync((void *)p_out, io + off_out, (size_t)nseq * od * 4,
                                            hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) rc = fail(FH_EHIP, "hipMemcpyAsync: %s", hipGetErrorString(e));
    }
    const int rc_end = end_on(m, s);
    const hipError_t es = hipStreamSynchronize(s);
    release_pacer(m, pacer);
    if (rc) return rc;
    if (rc_end) return rc_end;
    if (es != hipSuccess) return fail(FH_EHIP, "hipStreamSynchronize: %s", hipGetErrorString(es));
    for (int j = 0; j < nseq; j++) memcpy(out + (size_t)ord[(size_t)j] * od, p_out + (size_t)j * od, (size_t)od * 4);
    if (m->prof) drain_profile(m);
    return FH_OK;
}

extern "C" int fh_encode_device(fh_model *m, const int32_t *d_ids, const int32_t *d_offsets, int32_t nseq,
                                int32_t total_tokens, int32_t max_len, int32_t out_dim, float *d_out, void *stream,
                                const int32_t *h_offsets) {
    if (!m) return fail(FH_EINVAL, "native: null model");
    if (nseq <= 0) return nseq == 0 ? FH_OK : fail(FH_EINVAL, "native: negative batch size");
    if (!d_ids || !d_offsets || !d_out) return fail(FH_EINVAL, "native: null buffer");
    const fh_config &c = m->cfg;
    if (out_dim < 0 || out_dim > c.hidden_size || (out_dim != 0 && out_dim != c.hidden_size && !c.matryoshka))
        return fail(FH_EINVAL, "native: requested dim %d not supported", out_dim);
    if (max_len <= 0 || max_len > m->eff_max || total_tokens < nseq || total_tokens > (int64_t)nseq * max_len)
        return fail(FH_EINVAL, "native: inconsistent batch description (T=%d, nseq=%d, max_len=%d)", total_tokens,
                    nseq, max_len);
    std::lock_guard<std::mutex> lk(m->mu);
    HIPCHK(hipSetDevice(m->device));
    int rc = ensure_workspace(m, total_tokens, nseq);
    if (rc) return rc;
    BatchInfo b{d_ids, d_offsets, nseq, total_tokens, max_len, out_dim, d_out};
    if (h_offsets) {
        for (int i = 0; i < nseq; i++) {
            const double L = (double)(h_offsets[i + 1] - h_offsets[i]);
            b.sum_l2 += L * L;
        }
    } else {
        b.sum_l2 = (double)total_tokens * max_len;  // upper bound without host offsets
    }
    classify(b, h_offsets);
    hipStream_t s = stream ? (hipStream_t)stream : m->stream;
    if ((rc = begin_on(m, s))) return rc;
    rc = run_forward(m, b, s);
    const int rc_end = end_on(m, s);
    return rc ? rc : rc_end;
}

extern "C" int fh_encode_device_noalloc(fh_model *m, const int32_t *d_ids, const int32_t *d_offsets, int32_t nseq,
                                        int32_t total_tokens, int32_t max_len, int32_t out_dim, float *d_out,
                                        void *stream, const int32_t *h_offsets) {
    if (!m) return fail(FH_EINVAL, "native: null model");
    if (nseq <= 0) return nseq == 0 ? FH_OK : fail(FH_EINVAL, "native: negative batch size");
    if (!d_ids || !d_offsets || !d_out) return fail(FH_EINVAL, "native: null buffer");
    const fh_config &c = m->cfg;
    if (out_dim < 0 || out_dim > c.hidden_size || (out_dim != 0 && out_dim != c.hidden_size && !c.matryoshka))
        return fail(FH_EINVAL, "native: requested dim %d not supported", out_dim);
    if (max_len <= 0 || max_len > m->eff_max || total_tokens < nseq || total_tokens > (int64_t)nseq * max_len)
        return fail(FH_EINVAL, "native: inconsistent batch description (T=%d, nseq=%d, max_len=%d)", total_tokens,
                    nseq, max_len);
    std::lock_guard<std::mutex> lk(m->mu);
    HIPCHK(hipSetDevice(m->device));
    DevScratch &d = g_scratch[m->device];
    if (!d.ptr) return fail(FH_EHIP, "scratch of device %d not set up", m->device);
    const WsPlan plan = workspace_plan(m, total_tokens, nseq);
    const size_t need = workspace_bytes(plan);
    if (need > kScratchBytes)
        return fail(FH_EINVAL,
                    "native: batch of %d tokens in %d sequences needs %zu bytes of scratch; the no-allocation entry "
                    "point holds %zu (use fh_encode_device)",
                    total_tokens, nseq, need, kScratchBytes);
    BatchInfo b{d_ids, d_offsets, nseq, total_tokens, max_len, out_dim, d_out};
    if (h_offsets) {
        for (int i = 0; i < nseq; i++) {
            const double L = (double)(h_offsets[i + 1] - h_offsets[i]);
            b.sum_l2 += L * L;
        }
    }
    classify(b, h_offsets);
    // The model's buffers point into the scratch for this call only, and the
    // profiler (which creates events) is off for it.
    void *saved[20];
    for (int i = 0; i < plan.n; i++) saved[i] = *plan.e[i].first;
    const bool prof = m->prof;
    m->prof = false;
    carve(plan, (char *)d.ptr);
    hipStream_t s = stream ? (hipStream_t)stream : m->stream;
    int rc = FH_OK;
    {
        std::lock_guard<std::mutex> sl(g_scratch_mu);
        hipError_t e = d.used ? hipStreamWaitEvent(s, d.done, 0) : hipSuccess;
        if (e != hipSuccess) rc = fail(FH_EHIP, "hipStreamWaitEvent: %s", hipGetErrorString(e));
        if (rc == FH_OK) rc = run_forward(m, b, s);
        e = hipEventRecord(d.done, s);
        if (e == hipSuccess) d.used = true;
        else if (rc == FH_OK) rc = fail(FH_EHIP, "hipEventRecord: %s", hipGetErrorString(e));
    }
    for (int i = 0; i < plan.n; i++) *plan.e[i].first = saved[i];
    m->prof = prof;
    return rc;
}

extern "C" int64_t fh_noalloc_scratch_bytes(void) { return (int64_t)kScratchBytes; }

extern "C" int32_t fh_route_flags(int32_t hidden, int32_t inter, int32_t swiglu, int32_t M) {
    if (hidden <= 0 || inter <= 0 || M <= 0) return 0;
    const int H = hidden, I = inter;
    const bool fold = H % 64 == 0 && (H / 64 == 4 || H / 64 == 6 || H / 64 == 8 || H / 64 == 12 || H / 64 == 16);
    if (!fold) return 0;
    auto mat = [](int n, int k) {
        DevMat d;
        d.n = n;
        d.k = k;
        d.wr = (n % 128 == 0 && k % 64 == 0) ? (void *)&d : nullptr;  // a stand-in: only its presence is read
        return d;
    };
    auto args = [](int M, int n, int k, int lda, int ldc, bool resid) {
        GemmArgs g{};
        g.M = M;
        g.N = n;
        g.K = k;
        g.lda = lda;
        g.ldb = k;
        g.ldc = ldc;
        g.ldr = resid ? ldc : 0;
        g.resid_h = resid ? (const f16 *)&g : nullptr;  // presence only
        return g;
    };
    int32_t f = 0;
    const DevMat q = mat(3 * H, H), o = mat(H, H), f1 = mat(swiglu ? 2 * I : I, H), f2 = mat(H, I);
    if (use_ring(q, args(M, 3 * H, H, H, 3 * H, false), fh::ACT_NONE, false, fh::LN_IN)) f |= FH_ROUTE_RING_QKV;
    if (use_ring(o, args(M, H, H, H, H, true), fh::ACT_NONE, false, fh::RES_LN)) f |= FH_ROUTE_RING_OUT;
    if (swiglu ? use_ring(f1, args(M, 2 * I, H, H, I, false), fh::ACT_SWIGLU, false, fh::LN_IN)
               : use_ring(f1, args(M, I, H, H, I, false), fh::ACT_GELU, false, fh::LN_IN))
        f |= FH_ROUTE_RING_FFN1;
    if (use_ring(f2, args(M, H, I, I, H, true), fh::ACT_NONE, false, fh::RES_LN)) f |= FH_ROUTE_RING_FC2;
    if (!swiglu && fh::mlp_ok(1, H, I) && I % 128 == 0) {
        DevLayer L;
        L.fc2.wm = L.ffn1.wm = L.out.wm = (void *)&L;  // presence only
        L.fc2.n = H;
        if (use_mlp(L, M, I, false)) f |= FH_ROUTE_MLP;
        if (use_mlp(L, M, I, true)) f |= FH_ROUTE_MLP_QKV;
    }
    return f;
}

extern "C" int fh_profile_enable(fh_model *m, int32_t on) {
    if (!m) return fail(FH_EINVAL, "null model");
    std::lock_guard<std::mutex> lk(m->mu);
    m->prof = on != 0;
    return FH_OK;
}

extern "C" int fh_profile_reset(fh_model *m) {
    if (!m) return fail(FH_EINVAL, "null model");
    std::lock_guard<std::mutex> lk(m->mu);
    drain_profile(m);
    for (int i = 0; i < K_NCLASS; i++) {
        m->prof_ms[i] = m->prof_flops[i] = m->prof_bytes[i] = 0.0;
        m->prof_launches[i] = 0;
    }
    return FH_OK;
}

extern "C" int fh_profile_read(fh_model *m, const char **names, double *ms, int64_t *launches, double *flops,
                               double *bytes, int32_t cap) {
    if (!m) return fail(FH_EINVAL, "null model");
    std::lock_guard<std::mutex> lk(m->mu);
    drain_profile(m);
    const int n = std::min<int>(cap, K_NCLASS);
    for (int i = 0; i < n; i++) {
        if (names) names[i] = kClassNames[i];
        if (ms) ms[i] = m->prof_ms[i];
        if (launches) launches[i] = m->prof_launches[i];
        if (flops) flops[i] = m->prof_flops[i];
        if (bytes) bytes[i] = m->prof_bytes[i];
    }
    return K_NCLASS;
}
