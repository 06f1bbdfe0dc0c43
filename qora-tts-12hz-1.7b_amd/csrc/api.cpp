// api.cpp — host runtime behind the C-ABI (include/qtts.h): contexts, weight
// upload + repack, the device KV arena, and the enqueue sequences of the
// talker step, the predictor frame and the frame loop (replayed as a HIP
// graph).  Host code; every kernel it launches lives in kernels.hip.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <array>
#include <atomic>
#include <cstring>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "../../include/qtts.h"
#include "../../include/qtts_decoder.h"
#include "../../include/qtts_synth.h"
#include "engine.h"
#include "internal.h"

using namespace qtts;

namespace {

constexpr size_t kPartialFloats = (size_t)1 << 20;  // split-K partials
constexpr int kCounters = 8192;
constexpr size_t kAttnPartFloats = (size_t)4 << 20;
constexpr int kAttnCounters = 1024;

}  // namespace

struct qtts_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    float *partial = nullptr;
    unsigned *counters = nullptr;
    float *attn_part = nullptr;
    unsigned *attn_counters = nullptr;
    // staging for the stand-alone operators
    float *d_in = nullptr;
    size_t d_in_cap = 0;
    float *d_out = nullptr;
    size_t d_out_cap = 0;
    uint32_t *d_small = nullptr;  // tokens, prev tokens, status, rng (256 B)
    // persistent-kernel engine
    EngState *eng_state = nullptr;  // [2]
    int *eng_done = nullptr;
    tv_t *eng_bar = nullptr;  // [grid + 1] arrival words and the release word of the barrier between codes
    int *eng_status = nullptr;
    uint32_t eng_tag = 0;  // tag base of the last code launched
    uint32_t eng_epoch = 0;  // bumped when the tag space restarts (a program's arena is cleared before its next launch)
    int eng_grid = 0;
    uint64_t *eng_trace = nullptr;  // QTTS_ENGINE_TRACE: per-op block timestamps
    size_t eng_trace_cap = 0;
    long long eng_launches = 0;
    // MFMA GEMM scratch: the rows split into binary16 hi/lo, and K-chunk partials
    _Float16 *mfma_x = nullptr;
    size_t mfma_x_cap = 0;
    float *mfma_part = nullptr;
    size_t mfma_part_cap = 0;
    // The context and every object made from it hold one reference each, so
    // objects may be freed after qtts_ctx_destroy (e.g. in any order at
    // interpreter shutdown).
    std::atomic<int> refs{1};
};

namespace {

qtts_ctx *ctx_retain(qtts_ctx *c) {
    c->refs.fetch_add(1);
    return c;
}

void ctx_release(qtts_ctx *c) {
    if (c->refs.fetch_sub(1) != 1) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    (void)hipFree(c->partial);
    (void)hipFree(c->counters);
    (void)hipFree(c->attn_part);
    (void)hipFree(c->attn_counters);
    (void)hipFree(c->d_in);
    (void)hipFree(c->d_out);
    (void)hipFree(c->d_small);
    (void)hipFree(c->eng_state);
    (void)hipFree(c->eng_done);
    (void)hipFree(c->eng_bar);
    (void)hipFree(c->eng_trace);
    (void)hipFree(c->mfma_x);
    (void)hipFree(c->mfma_part);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

}  // namespace

struct qtts_q4 {
    qtts_ctx *ctx = nullptr;
    DevQ4 d{};
    void *mem = nullptr;
    size_t bytes = 0;
    DevQ4Mfma m{};  // MFMA operand copy, made by the first GEMM of >= 8 rows
    void *mfma_mem = nullptr;
    int mfma_state = 0;  // 0 not tried, 1 made, -1 the weight stays on the VALU path
};

// Serial numbers identify caches and predictors in the engine's program
// caches: a freed object's host address can be reused by the next one.
static std::atomic<uint64_t> g_serial{0};

struct qtts_kv {
    qtts_ctx *ctx = nullptr;
    uint64_t serial = ++g_serial;
    int layers = 0, kvh = 0, hd = 0, cap = 0, len = 0;
    float *k = nullptr, *v = nullptr;  // [layer][kvh][cap][hd]
    float *layer_k(int l) const { return k + (size_t)l * kvh * cap * hd; }
    float *layer_v(int l) const { return v + (size_t)l * kvh * cap * hd; }
};

namespace {

struct DevLayer {
    DevQ4 qkv{}, o{}, gu{}, down{};
    uint16_t *q_norm = nullptr, *k_norm = nullptr, *in_g = nullptr, *post_g = nullptr;
};

struct Stack {  // shapes shared by the talker and predictor layer stacks
    int layers = 0, hidden = 0, nq = 0, nkv = 0, hd = 0, inter = 0;
    std::vector<DevLayer> L;
    uint16_t *final_g = nullptr;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    int rope_rows = 0;
    int rope_skip_oob = 0;
};

qtts_status fail(qtts_ctx *c, qtts_status s, const std::string &m) {
    if (c) c->err = m;
    return s;
}

#define HIP_TRY(ctx, expr)                                                                   \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess)                                                                \
            return fail((ctx), QTTS_EDEVICE, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define QTTS_TRY(expr)                     \
    do {                                   \
        qtts_status s_ = (expr);           \
        if (s_ != QTTS_OK) return s_;      \
    } while (0)

qtts_status check_launch(qtts_ctx *c, const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(c, QTTS_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
    return QTTS_OK;
}

// Owns device allocations of a model object.
struct Owner {
    std::vector<void *> ptrs;
    ~Owner() {
        for (void *p : ptrs) (void)hipFree(p);
    }
    template <class T>
    qtts_status alloc(qtts_ctx *c, T **out, size_t count) {
        void *p = nullptr;
        hipError_t e = hipMalloc(&p, count * sizeof(T) > 0 ? count * sizeof(T) : 1);
        if (e != hipSuccess) return fail(c, QTTS_ENOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
        ptrs.push_back(p);
        *out = reinterpret_cast<T *>(p);
        return QTTS_OK;
    }
};

qtts_status check_view(qtts_ctx *c, const qtts_q4_view *v, int K, int N, const char *name) {
    if (!v || !v->packed || !v->scales) return fail(c, QTTS_EINVAL, std::string(name) + ": null weight");
    if (v->k != K || v->n != N || N % 32 != 0 || K <= 0)
        return fail(c, QTTS_ESHAPE, std::string(name) + ": shape " + std::to_string(v->k) + "x" +
                                        std::to_string(v->n) + ", expected " + std::to_string(K) + "x" +
                                        std::to_string(N));
    return QTTS_OK;
}

qtts_status alloc_q4(qtts_ctx *c, Owner &own, int K, int N, DevQ4 *d) {
    uint8_t *mem = nullptr;
    const size_t wbytes = (size_t)K * N / 2, sbytes = (size_t)K * (N / 32) * 2;
    QTTS_TRY(own.alloc(c, &mem, wbytes + sbytes));
    d->wq = reinterpret_cast<const uint4 *>(mem);
    d->ws = reinterpret_cast<const uint16_t *>(mem + wbytes);
    d->K = K;
    d->N = N;
    return QTTS_OK;
}

// Uploads one reference-layout weight into columns [col0, col0+n) of d.
qtts_status upload_part(qtts_ctx *c, const qtts_q4_view *v, const DevQ4 &d, int col0) {
    const size_t pb = (size_t)v->k * v->n / 2, sb = (size_t)v->k * (v->n / 32) * 2;
    uint8_t *stage = nullptr;
    HIP_TRY(c, hipMalloc(&stage, pb + sb));
    hipError_t e = hipMemcpyAsync(stage, v->packed, pb, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(stage + pb, v->scales, sb, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) {
        launch_repack_q4(c->stream, stage, reinterpret_cast<const uint16_t *>(stage + pb), v->k, v->n, col0, d.N,
                         const_cast<uint4 *>(d.wq), const_cast<uint16_t *>(d.ws));
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    (void)hipFree(stage);
    if (e != hipSuccess) return fail(c, QTTS_EDEVICE, std::string("weight upload: ") + hipGetErrorString(e));
    return QTTS_OK;
}

template <class T>
qtts_status upload_array(qtts_ctx *c, Owner &own, const T *src, size_t count, T **dst, const char *name) {
    if (!src) return fail(c, QTTS_EINVAL, std::string(name) + ": null");
    QTTS_TRY(own.alloc(c, dst, count));
    HIP_TRY(c, hipMemcpy(*dst, src, count * sizeof(T), hipMemcpyHostToDevice));
    return QTTS_OK;
}

// RoPE table exactly as build_mrope_tables (src/rope.rs:11-41) and the
// predictor table (src/loader.rs:859-874): double pow/cos/sin, cast to float.
// The first `rows` rows of the RoPE tables: the caller's (cos_in/sin_in,
// e.g. a model file's) or built from theta.
qtts_status upload_rope(qtts_ctx *c, Owner &own, int head_dim, int rows, double theta, const float *cos_in,
                        const float *sin_in, Stack *st) {
    const int half = head_dim / 2;
    if ((cos_in == nullptr) != (sin_in == nullptr)) return fail(c, QTTS_EINVAL, "RoPE tables: give both or neither");
    if (cos_in) {
        QTTS_TRY(upload_array(c, own, cos_in, (size_t)rows * half, &st->rope_cos, "rope cos"));
        QTTS_TRY(upload_array(c, own, sin_in, (size_t)rows * half, &st->rope_sin, "rope sin"));
        st->rope_rows = rows;
        return QTTS_OK;
    }
    std::vector<float> cs((size_t)rows * half), sn((size_t)rows * half);
    for (int i = 0; i < half; i++) {
        const double freq = 1.0 / std::pow(theta, (double)(2 * i) / (double)head_dim);
        for (int pos = 0; pos < rows; pos++) {
            const double angle = (double)pos * freq;
            cs[(size_t)pos * half + i] = (float)std::cos(angle);
            sn[(size_t)pos * half + i] = (float)std::sin(angle);
        }
    }
    QTTS_TRY(upload_array(c, own, cs.data(), cs.size(), &st->rope_cos, "rope cos"));
    QTTS_TRY(upload_array(c, own, sn.data(), sn.size(), &st->rope_sin, "rope sin"));
    st->rope_rows = rows;
    return QTTS_OK;
}

qtts_status upload_stack(qtts_ctx *c, Owner &own, int num_layers, const qtts_layer_view *layers, int hidden,
                         int nq, int nkv, int hd, Stack *st) {
    if (!layers || num_layers <= 0) return fail(c, QTTS_EINVAL, "no layers");
    if (hd != 128) return fail(c, QTTS_ESHAPE, "head_dim must be 128");
    if (nkv <= 0 || nq % nkv != 0 || nq / nkv > 4) return fail(c, QTTS_ESHAPE, "unsupported GQA grouping");
    const int inter = layers[0].gate_proj.n;
    st->layers = num_layers;
    st->hidden = hidden;
    st->nq = nq;
    st->nkv = nkv;
    st->hd = hd;
    st->inter = inter;
    st->L.resize(num_layers);
    const int qd = nq * hd, kd = nkv * hd;
    for (int l = 0; l < num_layers; l++) {
        const qtts_layer_view &v = layers[l];
        DevLayer &d = st->L[l];
        QTTS_TRY(check_view(c, &v.q_proj, hidden, qd, "q_proj"));
        QTTS_TRY(check_view(c, &v.k_proj, hidden, kd, "k_proj"));
        QTTS_TRY(check_view(c, &v.v_proj, hidden, kd, "v_proj"));
        QTTS_TRY(check_view(c, &v.o_proj, qd, hidden, "o_proj"));
        QTTS_TRY(check_view(c, &v.gate_proj, hidden, inter, "gate_proj"));
        QTTS_TRY(check_view(c, &v.up_proj, hidden, inter, "up_proj"));
        QTTS_TRY(check_view(c, &v.down_proj, inter, hidden, "down_proj"));
        // q|k|v and gate|up are concatenated along N: both splits fall on
        // 32-column scale-group boundaries, so every column's K-sum is the
        // reference's own.
        QTTS_TRY(alloc_q4(c, own, hidden, qd + 2 * kd, &d.qkv));
        QTTS_TRY(upload_part(c, &v.q_proj, d.qkv, 0));
        QTTS_TRY(upload_part(c, &v.k_proj, d.qkv, qd));
        QTTS_TRY(upload_part(c, &v.v_proj, d.qkv, qd + kd));
        QTTS_TRY(alloc_q4(c, own, qd, hidden, &d.o));
        QTTS_TRY(upload_part(c, &v.o_proj, d.o, 0));
        QTTS_TRY(alloc_q4(c, own, hidden, 2 * inter, &d.gu));
        QTTS_TRY(upload_part(c, &v.gate_proj, d.gu, 0));
        QTTS_TRY(upload_part(c, &v.up_proj, d.gu, inter));
        QTTS_TRY(alloc_q4(c, own, inter, hidden, &d.down));
        QTTS_TRY(upload_part(c, &v.down_proj, d.down, 0));
        QTTS_TRY(upload_array(c, own, v.q_norm, (size_t)hd, &d.q_norm, "q_norm"));
        QTTS_TRY(upload_array(c, own, v.k_norm, (size_t)hd, &d.k_norm, "k_norm"));
        QTTS_TRY(upload_array(c, own, v.input_norm_gamma, (size_t)hidden, &d.in_g, "input_norm_gamma"));
        QTTS_TRY(upload_array(c, own, v.post_attn_norm_gamma, (size_t)hidden, &d.post_g, "post_attn_norm_gamma"));
    }
    return QTTS_OK;
}

GemvParams gemv_base(qtts_ctx *c, const DevQ4 &w, int M) {
    GemvParams p{};
    p.w = w;
    p.M = M;
    plan_gemv(w.K, w.N, M, &p.kc, &p.rpt);
    p.partial = c->partial;
    p.counters = c->counters;
    return p;
}

qtts_status run_gemv(qtts_ctx *c, const GemvParams &p) {
    if ((size_t)p.kc * p.M * p.w.N > kPartialFloats || p.w.N / 32 + 1 > kCounters)
        return fail(c, QTTS_ESHAPE, "GEMV too large for the partial buffer");
    if (p.M < 1 || p.M > kMaxM) return fail(c, QTTS_EINVAL, "GEMV rows per launch out of range");
    launch_gemv(c->stream, p);
    return check_launch(c, "k_gemv");
}

// The MFMA operand copy of a panel-major weight (one allocation at *mem).
// *ok is false (and *mem null) for a weight the matrix-core path cannot take
// exactly: a shape off the 16 x 32 grid, K above the row prologue's limit,
// or a scale above 8188 in magnitude.  Synchronises the stream.
qtts_status make_mfma_copy(qtts_ctx *c, const DevQ4 &w, void **mem, DevQ4Mfma *m, bool *ok) {
    *mem = nullptr;
    *ok = false;
    if (w.K % 16 != 0 || w.N % 32 != 0 || w.K > kMfmaRowsMaxK) return QTTS_OK;
    const size_t nw = (size_t)(w.N / 32) * (w.K / 16) * 64, ns = (size_t)(w.N / 32) * w.K;
    const size_t flag_off = (nw * 4 + 2 * ns * 2 + 255) / 256 * 256;
    HIP_TRY(c, hipMalloc(mem, flag_off + 256));
    m->wm = reinterpret_cast<uint32_t *>(*mem);
    m->sa = reinterpret_cast<uint16_t *>((uint8_t *)*mem + nw * 4);
    m->sb = m->sa + ns;
    m->K = w.K;
    m->N = w.N;
    int *flag = reinterpret_cast<int *>((uint8_t *)*mem + flag_off);
    HIP_TRY(c, hipMemsetAsync(flag, 0, sizeof(int), c->stream));
    launch_repack_mfma(c->stream, w, const_cast<uint32_t *>(m->wm), const_cast<uint16_t *>(m->sa),
                       const_cast<uint16_t *>(m->sb), flag);
    QTTS_TRY(check_launch(c, "k_repack_mfma"));
    int too_large = 0;
    HIP_TRY(c, hipMemcpyAsync(&too_large, flag, sizeof(int), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    if (too_large) {
        (void)hipFree(*mem);
        *mem = nullptr;
        return QTTS_OK;
    }
    *ok = true;
    return QTTS_OK;
}

template <class T>
qtts_status grow(qtts_ctx *c, T **buf, size_t *cap, size_t need) {
    if (*cap >= need) return QTTS_OK;
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    (void)hipFree(*buf);
    *buf = nullptr;
    *cap = 0;
    HIP_TRY(c, hipMalloc(buf, need * sizeof(T)));
    *cap = need;
    return QTTS_OK;
}

// Steps per wave (sw) and K chunks (kc) of the MFMA GEMM for K rows.
void mfma_plan(int K, int *sw, int *kc) {
    const int Ks = K / 16;
    int s = 8;
    while (s > 1 && 4 * (s / 2) >= Ks) s /= 2;
    *sw = s;
    *kc = (Ks + 4 * s - 1) / (4 * s);
}

// Grows the MFMA GEMM scratch for a K x N weight at up to M rows, so that a
// later call allocates nothing (e.g. under stream capture).
qtts_status mfma_reserve(qtts_ctx *c, int K, int N, int M) {
    int sw, kc;
    mfma_plan(K, &sw, &kc);
    const int Mpad = M > 32 ? 64 : 32;
    QTTS_TRY(grow(c, &c->mfma_x, &c->mfma_x_cap, (size_t)2 * 64 * K + 2 * 64));
    if (kc > 1) QTTS_TRY(grow(c, &c->mfma_part, &c->mfma_part_cap, (size_t)kc * Mpad * N));
    return QTTS_OK;
}

// y[m] (+)= f(x[m]) . W (+ bias) for M rows on the matrix cores
// (csrc/mfma.hip), f the row prologue (MfmaRowsMode), 64 rows per pass: the
// prologue and binary16 split, then one block per (panel, K chunk) of
// 4 * sw 16-row steps, and the last block of a panel sums its chunks.  sw is
// 8 (each wave keeps 8 steps of operand loads in flight; measured fastest at
// every talker shape, 64 rows) unless K is short.
qtts_status run_gemm_mfma(qtts_ctx *c, const DevQ4Mfma &w, const float *x, int M, int ldx, int mode,
                          const uint16_t *gamma, float *y, int ldy, const float *bias, bool accumulate,
                          float *norm_out = nullptr, int ldn = 0) {
    const int K = w.K, N = w.N, panels = N / 32;
    if (K % 16 || N % 32 || K > kMfmaRowsMaxK || ldx % 4 || ((uintptr_t)x & 15))
        return fail(c, QTTS_ESHAPE, "MFMA GEMM: unsupported shape or unaligned rows");
    if (panels > kCounters) return fail(c, QTTS_ESHAPE, "MFMA GEMM: more panels than counters");
    int sw, kc;
    mfma_plan(K, &sw, &kc);
    for (int r0 = 0; r0 < M; r0 += 64) {
        const int Mc = M - r0 < 64 ? M - r0 : 64;
        const int mt = Mc > 32 ? 2 : 1, Mpad = 32 * mt;
        QTTS_TRY(grow(c, &c->mfma_x, &c->mfma_x_cap, (size_t)2 * 64 * K + 2 * 64));
        if (kc > 1) QTTS_TRY(grow(c, &c->mfma_part, &c->mfma_part_cap, (size_t)kc * Mpad * N));
        MfmaRowsParams r{};
        r.x = x + (size_t)r0 * ldx;
        r.ldx = ldx;
        r.K = K;
        r.M = Mc;
        r.Mpad = Mpad;
        r.mode = mode;
        r.gamma = gamma;
        r.xh = c->mfma_x;
        r.xl = c->mfma_x + (size_t)Mpad * K;
        r.rexp = reinterpret_cast<int *>(c->mfma_x + (size_t)2 * 64 * K);
        r.norm_out = norm_out ? norm_out + (size_t)r0 * ldn : nullptr;
        r.ldn = ldn;
        launch_mfma_rows(c->stream, r);
        QTTS_TRY(check_launch(c, "k_mfma_rows"));
        GemmMfmaParams p{};
        p.w = w;
        p.xh = r.xh;
        p.xl = r.xl;
        p.rexp = r.rexp;
        p.M = Mc;
        p.part = c->mfma_part;
        p.counters = c->counters;
        p.bias = bias;
        p.y = y + (size_t)r0 * ldy;
        p.ldy = ldy;
        p.accumulate = accumulate ? 1 : 0;
        launch_gemm_mfma(c->stream, p, mt, sw, kc);
        QTTS_TRY(check_launch(c, "k_gemm_mfma"));
    }
    return QTTS_OK;
}

int attn_nsplit(int cap, int min_split) {
    int n = (cap + kAttnMaxChunk - 1) / kAttnMaxChunk;
    if (n < min_split) n = min_split;
    return n;
}

// Splits of a one-row talker attention (k_attn): at least 16, and enough
// that a split holds <= 64 positions (its K and V rows then come in one
// round trip) up to 64 splits; past 64 * kAttnMaxChunk positions, as many
// as keep every split within the block's kAttnMaxChunk-entry score buffer.
int attn_nsplit_row(int cap) {
    int n = (cap + 63) / 64;
    if (n > 64) n = 64;
    if (n < 16) n = 16;
    const int fit = (cap + kAttnMaxChunk - 1) / kAttnMaxChunk;
    return n < fit ? fit : n;
}

// k_attn keeps a split's scores in a kAttnMaxChunk-entry LDS buffer per
// query head: a split of a cache of `cap` rows must not hold more.
bool attn_split_fits(int cap, int nsplit) { return nsplit > 0 && (cap + nsplit - 1) / nsplit <= kAttnMaxChunk; }

// One layer stack over M rows: QKV (RMSNorm prologue; QK-norm, RoPE and KV
// append epilogue) -> attention -> O (+residual) -> gate|up (RMSNorm
// prologue, SiLU*up epilogue) -> down (+residual).  Positions and cache rows
// come from d_pos/d_kvlen when given (graph replay), else the constants.
qtts_status enqueue_layers(qtts_ctx *c, const Stack &st, qtts_kv *kv, float *x, float *q, float *attn, float *h,
                           int M, const int *d_pos, int pos_const, const int *d_kvlen, int kvlen_const, int nsplit,
                           const int *d_done) {
    const int qd = st.nq * st.hd;
    for (int l = 0; l < st.layers; l++) {
        const DevLayer &Ly = st.L[l];
        float *kc = kv->layer_k(l), *vc = kv->layer_v(l);
        GemvParams p = gemv_base(c, Ly.qkv, M);
        p.prologue = PRO_RMSNORM;
        p.x = x;
        p.ldx = st.hidden;
        p.gamma = Ly.in_g;
        p.epilogue = EPI_QKV;
        p.y = q;
        p.ldy = qd;
        p.n_q_heads = st.nq;
        p.n_kv_heads = st.nkv;
        p.head_dim = st.hd;
        p.q_norm = Ly.q_norm;
        p.k_norm = Ly.k_norm;
        p.rope_cos = st.rope_cos;
        p.rope_sin = st.rope_sin;
        p.rope_rows = st.rope_rows;
        p.rope_skip_oob = st.rope_skip_oob;
        p.kcache = kc;
        p.vcache = vc;
        p.kv_cap = kv->cap;
        p.d_pos = d_pos;
        p.pos_const = pos_const;
        p.d_kvlen = d_kvlen;
        p.kvlen_const = kvlen_const;
        p.d_done = d_done;
        QTTS_TRY(run_gemv(c, p));

        AttnParams a{};
        a.q = q;
        a.ldq = qd;
        a.kcache = kc;
        a.vcache = vc;
        a.kv_cap = kv->cap;
        a.nq = st.nq;
        a.nkv = st.nkv;
        a.hd = st.hd;
        a.d_kvlen = d_kvlen;
        a.kvlen_const = kvlen_const;
        a.nsplit = nsplit;
        a.scale = 1.0f / sqrtf((float)st.hd);  // src/talker.rs:305
        a.part = c->attn_part;
        a.counters = c->attn_counters;
        a.out = attn;
        a.ldo = qd;
        a.d_done = d_done;
        if ((size_t)M * st.nq * nsplit * (st.hd + 2) > kAttnPartFloats || M * st.nkv > kAttnCounters)
            return fail(c, QTTS_ESHAPE, "attention split buffer too small");
        if (!attn_split_fits(kv->cap, nsplit)) return fail(c, QTTS_ESHAPE, "attention: a split exceeds the score buffer");
        launch_attention(c->stream, a, M);
        QTTS_TRY(check_launch(c, "k_attn"));

        p = gemv_base(c, Ly.o, M);
        p.prologue = PRO_PLAIN;
        p.x = attn;
        p.ldx = qd;
        p.epilogue = EPI_RESID;
        p.y = x;
        p.ldy = st.hidden;
        p.d_done = d_done;
        QTTS_TRY(run_gemv(c, p));

        p = gemv_base(c, Ly.gu, M);
        p.prologue = PRO_RMSNORM;
        p.x = x;
        p.ldx = st.hidden;
        p.gamma = Ly.post_g;
        p.epilogue = EPI_SWIGLU;
        p.y = h;
        p.ldy = st.inter;
        p.d_done = d_done;
        QTTS_TRY(run_gemv(c, p));

        p = gemv_base(c, Ly.down, M);
        p.prologue = PRO_PLAIN;
        p.x = h;
        p.ldx = st.inter;
        p.epilogue = EPI_RESID;
        p.y = x;
        p.ldy = st.hidden;
        p.d_done = d_done;
        QTTS_TRY(run_gemv(c, p));
    }
    return QTTS_OK;
}

qtts_status ensure_staging(qtts_ctx *c, size_t in_floats, size_t out_floats) {
    if (in_floats > c->d_in_cap) {
        if (c->d_in) (void)hipFree(c->d_in);
        c->d_in = nullptr;
        c->d_in_cap = 0;
        HIP_TRY(c, hipMalloc(&c->d_in, in_floats * sizeof(float)));
        c->d_in_cap = in_floats;
    }
    if (out_floats > c->d_out_cap) {
        if (c->d_out) (void)hipFree(c->d_out);
        c->d_out = nullptr;
        c->d_out_cap = 0;
        HIP_TRY(c, hipMalloc(&c->d_out, out_floats * sizeof(float)));
        c->d_out_cap = out_floats;
    }
    return QTTS_OK;
}

qtts_status sync(qtts_ctx *c) {
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return check_launch(c, "stream");
}

}  // namespace

namespace qtts {

struct TvRef {
    tv_t *p = nullptr;
    int tag = 0;
    int ld = 0;       // row stride
    int parts = 1;    // 2: each row is two parts of ld / 2 values to be added (a split_out GEMV)
};

// A program and its tagged-value arena.  Built twice: a sizing pass with null
// pointers, then the real pass into an arena of the measured size.
struct EngProgram {
    std::vector<EngOp> ops;
    EngOp *d_ops = nullptr;
    tv_t *arena = nullptr;
    size_t used = 0;
    uint32_t epoch = 0;  // the context's tag epoch the arena was last cleared in
    bool sizing = true;
    int next_tag = 1;
    int rot_next = 0;
    int grid = 1;
    const char *err = nullptr;  // set when an op cannot be expressed
    // Rotation plan: ops pushed while `rot_record` is set append their
    // rotation to it; while `rot_plan` is set they take theirs from it in
    // order (a repeated sequence of ops then lands on the same blocks).
    std::vector<int> *rot_record = nullptr;
    const std::vector<int> *rot_plan = nullptr;
    size_t plan_pos = 0;
    std::vector<int> lds_owner;  // block -> layer whose K/V rows it keeps in LDS (-1: none)
    // an op the kernel does not run (the caller takes the multi-kernel path)
    bool unsupported = false;
    ~EngProgram() {
        if (d_ops) (void)hipFree(d_ops);
        if (arena) (void)hipFree(arena);
    }
    void reset_build() {
        err = nullptr;
        rot_record = nullptr;
        rot_plan = nullptr;
        plan_pos = 0;
        lds_owner.assign((size_t)grid, -1);
        unsupported = false;
        ops.clear();
        used = 0;
        next_tag = 1;
        rot_next = 0;
    }
    tv_t *tv(size_t n) {
        const size_t off = used;
        used += (n + 31) & ~size_t(31);
        return sizing ? nullptr : arena + off;
    }
    int tag() { return next_tag++; }
    // The rotation the next op gets (from the plan, else the running one).
    int next_rot() const { return rot_plan && plan_pos < rot_plan->size() ? (*rot_plan)[plan_pos] : rot_next; }
    void push(EngOp &op) {
        op.rot = next_rot();
        if (rot_plan) plan_pos++;
        if (rot_record) rot_record->push_back(op.rot);
        rot_next = (op.rot + op.ntasks) % grid;
        ops.push_back(op);
    }
    // Blocks rot .. rot+n-1 keep layer l's K/V rows in LDS: true if they
    // are free (and are claimed) or already layer l's.
    bool claim_lds(int rot, int n, int l) {
        if (n > grid) return false;
        for (int i = 0; i < n; i++) {
            const int o = lds_owner[(size_t)((rot + i) % grid)];
            if (o != -1 && o != l) return false;
        }
        for (int i = 0; i < n; i++) lds_owner[(size_t)((rot + i) % grid)] = l;
        return true;
    }
};

}  // namespace qtts

// ===========================================================================
// Model objects
// ===========================================================================
struct qtts_talker {
    qtts_ctx *ctx = nullptr;
    Owner own;
    Stack st;
    int vocab = 0, max_pos = 0, nsplit = 16;
    DevQ4 head{}, emb{};
    float *x = nullptr, *q = nullptr, *attn = nullptr, *h = nullptr, *out = nullptr;
    LoopState *state = nullptr;
    // prefill work buffers
    float *xp = nullptr, *qp = nullptr, *ap = nullptr, *hp = nullptr, *rawp = nullptr;
    int prefill_cap = 0;
    std::vector<void *> prefill_bufs;
    // MFMA operand copies of the layer weights (qkv, o, gu, down per layer),
    // made by the first prefill of >= kMfmaMinRows rows
    std::vector<DevQ4Mfma> mfma;
    int mfma_state = 0;  // 0 not tried, 1 made, -1 some weight cannot use the matrix cores
    DevQ4Mfma head_mfma{};  // codec head, for the batched loop
    int head_mfma_state = 0;
    // loop buffers
    uint32_t *codes = nullptr;
    size_t codes_cap = 0;
    float *trailing = nullptr;
    size_t trailing_cap = 0;
    float *pad = nullptr;
    // prompt assembly (qtts_talker_text_upload): text embedding and the
    // two-layer text projection, and their work rows
    DevQ4 text_emb{}, fc1{}, fc2{};
    float *fc1_b = nullptr, *fc2_b = nullptr;
    int text_hidden = 0, has_text = 0;
    float *tx_raw = nullptr, *tx_h = nullptr, *tx_rows = nullptr;
    float *pr_codec = nullptr;  // [8][hidden]: the prompt's codec rows and the voice row
    uint32_t *tx_tok = nullptr;
    int tx_cap = 0;
    // prefill_talker's per-row token ids and text slots: [pf_cap] + [pf_cap]
    uint32_t *pf_tok = nullptr;
    int pf_cap = 0;
    // engine programs (built lazily, cached per cache object)
    std::unique_ptr<EngProgram> step_prog, frame_prog;
    uint64_t step_kv = 0;  // serial of the cache step_prog was built for
    std::string frame_key;
    ~qtts_talker() {
        for (void *p : prefill_bufs) (void)hipFree(p);
        if (codes) (void)hipFree(codes);
        if (trailing) (void)hipFree(trailing);
        for (void *p : {(void *)tx_raw, (void *)tx_h, (void *)tx_rows, (void *)tx_tok, (void *)pf_tok})
            if (p) (void)hipFree(p);
    }
};

struct qtts_predictor {
    qtts_ctx *ctx = nullptr;
    uint64_t serial = ++g_serial;
    Owner own;
    Stack st;
    int talker_hidden = 0, groups = 0, vocab = 0, embed_dim = 0, max_pos = 0;
    bool identity_proj = false;
    DevQ4 in_proj{};
    float *bias = nullptr;
    DevQ4 emb[kMaxGroups]{};
    DevQ4 heads[kMaxGroups]{};
    float *in2 = nullptr;  // [2][talker_hidden]: talker hidden, semantic embedding
    float *x2 = nullptr, *q2 = nullptr, *a2 = nullptr, *h2 = nullptr, *logits = nullptr;
    uint32_t *codes = nullptr;  // [16]
    int *status = nullptr;
    std::unique_ptr<EngProgram> prog;
    uint64_t prog_kv = 0;  // serial of the cache prog was built for
    // MFMA operand copies for the batched loop: 4 per layer, the input
    // projection, the heads (made by the first batched call)
    std::vector<DevQ4Mfma> mfma;
    DevQ4Mfma mfma_in{};
    std::vector<DevQ4Mfma> mfma_heads;
    int mfma_state = 0;  // 0 not tried, 1 made, -1 a weight cannot use the matrix cores
    // in_proj(emb[g][code]) + bias for every code of emb[0 .. groups-2]:
    // [groups-1][tab_rows][hidden], the engine's pass inputs by code
    float *tab = nullptr;
    int tab_rows = 0;
    int tab_state = 0;  // 0 not tried, 1 made, -1 not used
    // layer 0's raw q|k|v of every tab row, rms_norm_f16 with its input gamma
    // first: [groups-1][tab_rows][nq*hd + 2*nkv*hd] (with tab_state == 1)
    float *qkv_tab = nullptr;
};

// ===========================================================================
// Engine programs (host side of engine.hip)
// ===========================================================================
namespace {

EngInput in_tv(const TvRef &r, int row) {
    EngInput i{};
    i.kind = EIN_TV;
    i.tv = r.p ? r.p + (size_t)row * r.ld : nullptr;
    i.tag = r.tag;
    i.parts = r.parts;
    return i;
}
EngInput in_plain(const float *p) {
    EngInput i{};
    i.kind = EIN_PLAIN;
    i.plain = p;
    return i;
}
EngInput in_embed(const DevQ4 &emb, const TvRef &tok) {
    EngInput i{};
    i.kind = EIN_EMBED;
    i.emb = emb;
    i.tok_tv = tok.p;
    i.tag = tok.tag;
    return i;
}

// A layer input read from a per-code table at the argmax of a logits row:
// table[argmax(logits)], the argmax step's own code published as `code`.
struct TabIn {
    TvRef logits;
    int n = 0;
    const float *table = nullptr;
    int rows = 0;
    TvRef code;
    const float *qkv_table = nullptr;  // with it, the layer's raw q|k|v row by code too (no QKV step)
};

EngInput in_argtab(const TabIn &t) {
    EngInput i{};
    i.kind = EIN_ARGTAB;
    i.tv = t.logits.p;
    i.tag = t.logits.tag;
    i.n = t.n;
    i.table = t.table;
    i.table_rows = t.rows;
    return i;
}

struct GemvSpec {
    int M = 1;
    int epi = EEPI_STORE;
    bool norm = false;
    const uint16_t *gamma = nullptr;
    EngInput in[kEngMaxM]{};
    const float *bias = nullptr;
    TvRef resid{};
    const TabIn *resid_tab = nullptr;  // EEPI_RESID: the residual is the table row instead
    bool split_out = false;  // two K chunks publish as two output parts (when the shapes allow)
    int kc = 0;  // 0: choose
    float *out_plain = nullptr;
    float *norm_plain = nullptr;
};

TvRef add_gemv(EngProgram &P, const DevQ4 &w, const GemvSpec &sp) {
    EngOp op{};
    op.kind = EOP_GEMV;
    EngGemv &g = op.gemv;
    const int Nout = sp.epi == EEPI_SWIGLU ? w.N / 2 : w.N;
    // Tasks of whole 32-column panels (the kernel's GEMV slice width), or of
    // half panels for a SwiGLU step whose half-panel tasks fit the grid.
    const int NP = sp.epi == EEPI_SWIGLU ? 2 : 1;
    const char *half_env = std::getenv("QTTS_ENGINE_SWIGLU_COLS");
    auto half_fits = [&](int rows) {
        return NP == 2 && !(half_env && std::atoi(half_env) == 32) &&
               (Nout / 16) * ((w.K + kEngThreads * eng_rows_per_thread(16, 2) - 1) /
                              (kEngThreads * eng_rows_per_thread(16, 2))) * rows <= P.grid;
    };
    const bool half = half_fits(sp.M);
    const int C = half ? 16 : 32;
    const int rpt = eng_rows_per_thread(C, NP);
    if (Nout % 32 != 0 || (sp.norm && w.K > kEngThreads * kEngNormRows)) P.err = "engine GEMV shape not supported";
    // One K chunk where the rows fit one task: a split-K owner waits a
    // cross-block round trip for its partials.
    int kc = sp.kc > 0 ? sp.kc : 1;
    const int kmin = (w.K + kEngThreads * rpt - 1) / (kEngThreads * rpt);
    if (kc < kmin) kc = kmin;
    int kchunk = (w.K + kc - 1) / kc;
    kchunk = (kchunk + kEngThreads - 1) / kEngThreads * kEngThreads;
    kc = (w.K + kchunk - 1) / kchunk;
    if (sp.norm && kc != 1) P.err = "engine GEMV shape not supported";
    for (int m = 0; m < sp.M; m++)
        if (sp.in[m].kind == EIN_ARGTAB && (sp.M != 1 || NP != 1 || !sp.norm || sp.in[m].n > kEngArgtabMax))
            P.err = "engine table input not supported";
    if (sp.resid_tab && sp.M != 1) P.err = "engine table residual not supported";
    constexpr int kPartsMaxK = kEngThreads * kEngNormRows / 2;  // a normed input read in two parts
    for (int m = 0; m < sp.M; m++)
        if (sp.in[m].kind == EIN_TV && sp.in[m].parts == 2 && (!sp.norm || w.K > kPartsMaxK))
            P.err = "engine two-part input not supported";
    // Two K chunks publish their sums as two parts of the output (chunk 0
    // with the residual), so no block waits for the other's partial; the
    // consumers (normed GEMV inputs, residuals) add the parts.  (Three parts,
    // for the talker's down projection, measured slower: the wider poll costs
    // the whole kernel registers.)
    const bool split = sp.split_out && kc == 2 && NP == 1 && !sp.out_plain && !sp.norm_plain &&
                       Nout <= kPartsMaxK && sp.epi == EEPI_RESID && !sp.resid_tab;
    g.w = w;
    g.M = sp.M;
    g.kc = kc;
    g.kchunk = kchunk;
    g.cols = C;
    g.epi = sp.epi;
    g.norm = sp.norm ? 1 : 0;
    g.gamma = sp.gamma;
    for (int m = 0; m < kEngMaxM; m++) g.in[m] = sp.in[m];
    g.bias = sp.bias;
    g.resid = sp.resid.p;
    g.resid_tag = sp.resid.tag;
    g.ld_resid = sp.resid.ld;
    g.resid_parts = sp.resid.parts;
    if (sp.resid_tab) {
        g.resid_table = sp.resid_tab->table;
        g.resid_code = sp.resid_tab->code.p;
        g.resid_tag = sp.resid_tab->code.tag;
        g.resid_table_rows = sp.resid_tab->rows;
        g.ld_resid = Nout;
    }
    g.split_out = split ? 1 : 0;
    g.out = P.tv((size_t)sp.M * (split ? 2 : 1) * Nout);
    g.out_tag = P.tag();
    g.ld_out = split ? 2 * Nout : Nout;
    g.out_plain = sp.out_plain;
    g.ld_plain = Nout;
    g.norm_plain = sp.norm_plain;
    if (kc > 1 && !split) {
        g.part = P.tv((size_t)(kc - 1) * sp.M * w.N);
        g.part_tag = P.tag();
    }
    op.ntasks = (Nout / C) * kc * sp.M;  // one-row tasks for every row
    P.push(op);
    if (sp.M > 1 && P.rot_record && !P.rot_plan) {
        // The predictor's first pass (two rows) records the rotations its
        // one-row passes replay: the next op goes right after the blocks
        // this op has in those passes, so consecutive ops there run on
        // disjoint blocks and wait for their inputs from the start.
        P.rot_next = (op.rot + (Nout / (half_fits(1) ? 16 : 32)) * kc) % P.grid;
    }
    return TvRef{g.out, g.out_tag, g.ld_out, split ? 2 : 1};
}

TvRef add_attention(EngProgram &P, const Stack &st, int l, qtts_kv *kv, int M, const TvRef &qkv, bool from_state,
                    int pos_const, int len_const, int nsplit, const TabIn *qtab = nullptr) {
    EngOp op{};
    op.kind = EOP_ATTN;
    EngAttn &a = op.attn;
    a.qkv = qkv.p;
    a.qkv_tag = qkv.tag;
    a.ld_qkv = qkv.ld;
    a.M = M;
    a.nq = st.nq;
    a.nkv = st.nkv;
    a.hd = st.hd;
    a.q_norm = st.L[l].q_norm;
    a.k_norm = st.L[l].k_norm;
    a.rope_cos = st.rope_cos;
    a.rope_sin = st.rope_sin;
    a.rope_rows = st.rope_rows;
    a.rope_skip_oob = st.rope_skip_oob;
    a.kcache = kv->layer_k(l);
    a.vcache = kv->layer_v(l);
    a.kv_cap = kv->cap;
    a.from_state = from_state ? 1 : 0;
    a.pos_const = pos_const;
    a.len_const = len_const;
    a.nsplit = nsplit;
    // A short in-launch cache (the predictor) stays in the LDS of the blocks
    // that run this layer's steps, when those blocks serve no other layer
    // (the caller repeats each step's rotations).
    const bool lds_kv = !from_state && nsplit == 1 && st.hd == 128 && M * (st.nq / st.nkv) <= 4 &&
                        kv->cap <= kEngLdsKvPos && P.claim_lds(P.next_rot(), st.nkv, l);
    a.lds_kv = lds_kv ? 1 : 0;
    // outside LDS the kernel's attention serves at most two (row, q head)
    // pairs per kv head: the talker step (one row, 16 / 8 heads) and the
    // predictor's one-row steps; other shapes take the multi-kernel path
    if (!lds_kv && M * (st.nq / st.nkv) > 2) P.unsupported = true;
    if (qtab) {
        if (!lds_kv || M != 1 || qtab->n > kEngArgtabMax) P.err = "engine q|k|v table needs the LDS-resident attention";
        a.qkv = nullptr;
        a.ld_qkv = st.nq * st.hd + 2 * st.nkv * st.hd;
        a.qkv_table = qtab->qkv_table;
        a.qkv_table_rows = qtab->rows;
        a.logits = qtab->logits.p;
        a.logits_tag = qtab->logits.tag;
        a.logits_n = qtab->n;
    }
    a.scale = 1.0f / sqrtf((float)st.hd);  // src/talker.rs:305
    const int qd = st.nq * st.hd;
    TvRef out{};
    if (nsplit > 1) {
        a.part = P.tv((size_t)M * st.nq * nsplit * (st.hd + 2));
        a.part_tag = P.tag();
    } else {
        a.out = P.tv((size_t)M * qd);
        a.out_tag = P.tag();
    }
    op.ntasks = st.nkv * nsplit;
    if (nsplit == 1) out = TvRef{a.out, a.out_tag, qd};
    P.push(op);
    if (nsplit > 1) {
        EngOp cop{};
        cop.kind = EOP_COMBINE;
        EngCombine &cb = cop.comb;
        cb.part = a.part;
        cb.part_tag = a.part_tag;
        cb.M = M;
        cb.nq = st.nq;
        cb.hd = st.hd;
        cb.nsplit = nsplit;
        cb.out = P.tv((size_t)M * qd);
        cb.out_tag = P.tag();
        cop.ntasks = M * st.nq;
        P.push(cop);
        out = TvRef{cb.out, cb.out_tag, qd};
    }
    return out;
}

// One transformer layer over M rows; returns the new residual stream.  The
// input is x, or (tin, M == 1) the table row at the argmax of a logits row.
TvRef add_layer(EngProgram &P, const Stack &st, int l, qtts_kv *kv, int M, const TvRef &x, bool from_state,
                int pos_const, int len_const, int nsplit, const TabIn *tin = nullptr) {
    const DevLayer &L = st.L[l];
    GemvSpec q;
    q.M = M;
    q.norm = true;
    q.gamma = L.in_g;
    for (int m = 0; m < M; m++) q.in[m] = tin ? in_argtab(*tin) : in_tv(x, m);
    const bool qtab = tin && tin->qkv_table;  // the q|k|v row by code: no QKV step
    const TvRef qkv = qtab ? TvRef{} : add_gemv(P, L.qkv, q);
    const TvRef att = add_attention(P, st, l, kv, M, qkv, from_state, pos_const, len_const, nsplit, qtab ? tin : nullptr);
    GemvSpec o;
    o.M = M;
    for (int m = 0; m < M; m++) o.in[m] = in_tv(att, m);
    o.epi = EEPI_RESID;
    o.resid = x;
    o.resid_tab = tin;
    if (!tin && st.hidden <= kEngThreads * kEngNormRows / 2 && L.o.K >= 2 * kEngThreads) {
        // Two K chunks published as two output parts (the consumers, a normed
        // input and a residual, add them): the predictor's O projection
        // (2048 -> 1024) runs as 64 tasks instead of 32, 468.0 -> 469.7
        // codes/s.  A wider output's two-part normed input would need a wider
        // poll in the kernel.
        o.split_out = true;
        o.kc = 2;
    }
    const TvRef xm = add_gemv(P, L.o, o);
    GemvSpec gu;
    gu.M = M;
    gu.norm = true;
    gu.gamma = L.post_g;
    gu.epi = EEPI_SWIGLU;
    for (int m = 0; m < M; m++) gu.in[m] = in_tv(xm, m);
    const TvRef h = add_gemv(P, L.gu, gu);
    GemvSpec dn;
    dn.M = M;
    dn.epi = EEPI_RESID;
    dn.resid = xm;
    dn.split_out = true;
    for (int m = 0; m < M; m++) dn.in[m] = in_tv(h, m);
    return add_gemv(P, L.down, dn);
}

TvRef add_argmax(EngProgram &P, const TvRef &logits, int n, int group) {
    EngOp op{};
    op.kind = EOP_ARGMAX;
    op.ntasks = 1;
    op.amax.logits = logits.p;
    op.amax.logits_tag = logits.tag;
    op.amax.n = n;
    op.amax.code = P.tv(1);
    op.amax.code_tag = P.tag();
    op.amax.group = group;
    P.push(op);
    return TvRef{op.amax.code, op.amax.code_tag, 1};
}

TvRef add_embsum(EngProgram &P, int mode, const DevQ4 *codec_emb, const DevQ4 *group_emb, const TvRef *codes,
                 int groups, const TvRef &tok, const float *trailing, int trailing_len, const float *pad, int hidden) {
    EngOp op{};
    op.kind = EOP_EMBSUM;
    EngEmbSum &e = op.emb;
    e.mode = mode;
    if (codec_emb) e.codec_emb = *codec_emb;
    e.num_groups = groups;
    for (int g = 0; g < groups; g++) {
        e.group_emb[g] = group_emb[g];
        e.code[g] = codes[g].p;
        e.code_tag[g] = codes[g].tag;
    }
    e.tok = tok.p;
    e.tok_tag = tok.tag;
    e.trailing = trailing;
    e.trailing_len = trailing_len;
    e.pad = pad;
    e.hidden = hidden;
    e.out = P.tv((size_t)hidden);
    e.out_tag = P.tag();
    op.ntasks = (hidden + kEngThreads - 1) / kEngThreads;
    P.push(op);
    return TvRef{e.out, e.out_tag, hidden};
}

}  // namespace

// ===========================================================================
// Engine launches
// ===========================================================================
namespace {

bool engine_enabled() {
    const char *e = std::getenv("QTTS_ENGINE");
    return !(e && std::strcmp(e, "ops") == 0);
}

qtts_status eng_init(qtts_ctx *c) {
    if (c->eng_state) return QTTS_OK;
    HIP_TRY(c, hipMalloc(&c->eng_state, 2 * sizeof(EngState)));
    HIP_TRY(c, hipMalloc(&c->eng_done, 2 * sizeof(int)));
    c->eng_status = c->eng_done + 1;
    HIP_TRY(c, hipMemset(c->eng_done, 0, 2 * sizeof(int)));
    c->eng_grid = engine_max_grid();
    if (c->eng_grid <= 0) return fail(c, QTTS_EDEVICE, "engine kernel cannot be resident on this device");
    HIP_TRY(c, hipMalloc(&c->eng_bar, (size_t)(c->eng_grid + 1) * sizeof(tv_t)));
    HIP_TRY(c, hipMemset(c->eng_bar, 0, (size_t)(c->eng_grid + 1) * sizeof(tv_t)));
    c->eng_tag = 0;
    // QTTS_ENGINE_TAG_START=n (a test aid): the tag space starts at n, so that
    // a short run reaches its restart
    if (const char *e = std::getenv("QTTS_ENGINE_TAG_START")) {
        const unsigned long long v = std::strtoull(e, nullptr, 0);
        if (v < 0xFFFFFFFFull) c->eng_tag = (uint32_t)v;
    }
    return QTTS_OK;
}

using BuildFn = std::function<qtts_status(EngProgram &)>;

qtts_status eng_build(qtts_ctx *c, EngProgram &P, const BuildFn &fn) {
    P.grid = c->eng_grid;
    P.sizing = true;
    P.reset_build();
    QTTS_TRY(fn(P));
    if (P.err) return fail(c, QTTS_ESHAPE, P.err);
    if (P.unsupported) return QTTS_OK;  // nothing allocated; the caller checks
    const size_t need = P.used;
    if (P.arena) (void)hipFree(P.arena);
    if (P.d_ops) (void)hipFree(P.d_ops);
    P.arena = nullptr;
    P.d_ops = nullptr;
    HIP_TRY(c, hipMalloc(&P.arena, (need ? need : 1) * sizeof(tv_t)));
    HIP_TRY(c, hipMemset(P.arena, 0, (need ? need : 1) * sizeof(tv_t)));
    P.epoch = c->eng_epoch;
    P.sizing = false;
    P.reset_build();
    QTTS_TRY(fn(P));
    if ((uint32_t)P.next_tag >= kTagStride) return fail(c, QTTS_ESHAPE, "engine program has too many tagged outputs");
    HIP_TRY(c, hipMalloc(&P.d_ops, P.ops.size() * sizeof(EngOp)));
    HIP_TRY(c, hipMemcpy(P.d_ops, P.ops.data(), P.ops.size() * sizeof(EngOp), hipMemcpyHostToDevice));
    return QTTS_OK;
}

// Resets the abort word, status and both state copies.
qtts_status eng_reset(qtts_ctx *c, int pos, int kvlen, uint64_t rng) {
    EngState s[2];
    for (auto &x : s) {
        x.pos = pos;
        x.kvlen = kvlen;
        x.frame = 0;
        x.pad = 0;
        x.rng = rng;
    }
    HIP_TRY(c, hipMemcpyAsync(c->eng_state, s, sizeof(s), hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipMemsetAsync(c->eng_done, 0, 2 * sizeof(int), c->stream));
    return QTTS_OK;
}

// Runs `ncodes` codes of program P in one cooperative launch (a traced
// launch runs one code); code f reads state copy (st_in + f) & 1.
qtts_status eng_launch(qtts_ctx *c, EngProgram &P, int st_in, uint32_t *codes, int max_codes, int ncodes = 1) {
    const char *trace_env = std::getenv("QTTS_ENGINE_TRACE");
    const char *codes_env = std::getenv("QTTS_ENGINE_CODES");
    // (the barrier between codes waits on at most 256 blocks' words)
    const int per = P.grid > 256 ? 1 : codes_env ? std::max(1, std::atoi(codes_env)) : kEngCodesPerLaunch;
    if (ncodes > 1 && ((trace_env && *trace_env) || per < ncodes)) {
        const int step = (trace_env && *trace_env) ? 1 : per;
        for (int f = 0; f < ncodes; f += step)
            QTTS_TRY(eng_launch(c, P, (st_in + f) & 1, codes, max_codes, std::min(step, ncodes - f)));
        return QTTS_OK;
    }
    if (ncodes < 1) return QTTS_OK;
    if (c->eng_tag > 0xFFFFFFFFu - (uint32_t)(ncodes + 1) * kTagStride) {
        // The 32-bit tags are about to wrap (every 2^32 / kTagStride = 524,288
        // codes): once every launch has finished, restart them at zero in a
        // new epoch.  Every tagged word is cleared before the new tags are
        // used -- the barrier's words here, each program's arena before its
        // first launch of the epoch -- so no stale word carries a tag the new
        // epoch will wait for.
        HIP_TRY(c, hipStreamSynchronize(c->stream));
        HIP_TRY(c, hipMemsetAsync(c->eng_bar, 0, (size_t)(c->eng_grid + 1) * sizeof(tv_t), c->stream));
        c->eng_tag = 0;
        c->eng_epoch++;
    }
    if (P.epoch != c->eng_epoch) {
        HIP_TRY(c, hipMemsetAsync(P.arena, 0, (P.used ? P.used : 1) * sizeof(tv_t), c->stream));
        P.epoch = c->eng_epoch;
    }
    EngArgs a{};
    a.ops = P.d_ops;
    a.nops = (int)P.ops.size();
    a.tag_base = c->eng_tag + kTagStride;
    c->eng_tag += (uint32_t)ncodes * kTagStride;
    a.st = c->eng_state;
    a.st0 = st_in;
    a.ncodes = ncodes;
    a.bar = c->eng_bar;
    a.done = c->eng_done;
    a.status = c->eng_status;
    a.codes = codes;
    a.max_codes = max_codes;
    // QTTS_ENGINE_TRACE=<file>: each launch (from the QTTS_ENGINE_TRACE_FROM-th
    // of this context on) synchronizes and appends
    // {nops, grid, kind[nops], ntasks[nops], u64 stamps[nops][grid][kTraceSlots]}.
    const char *trace_path = std::getenv("QTTS_ENGINE_TRACE");
    const char *trace_from = std::getenv("QTTS_ENGINE_TRACE_FROM");
    const size_t trace_n = (size_t)a.nops * P.grid * kTraceSlots;
    const bool trace_this = trace_path && *trace_path && c->eng_launches >= (trace_from ? std::atoll(trace_from) : 0);
    c->eng_launches++;
    if (trace_this) {
        if (c->eng_trace_cap < trace_n) {
            if (c->eng_trace) (void)hipFree(c->eng_trace);
            c->eng_trace = nullptr;
            c->eng_trace_cap = 0;
            HIP_TRY(c, hipMalloc(&c->eng_trace, trace_n * sizeof(uint64_t)));
            c->eng_trace_cap = trace_n;
        }
        HIP_TRY(c, hipMemsetAsync(c->eng_trace, 0, trace_n * sizeof(uint64_t), c->stream));
        a.trace = c->eng_trace;
    }
    const char *launch_env = std::getenv("QTTS_ENGINE_LAUNCH");
    const bool coop = !(launch_env && std::strcmp(launch_env, "plain") == 0);
    hipError_t e = launch_engine(c->stream, a, P.grid, coop);
    if (e != hipSuccess) return fail(c, QTTS_EDEVICE, std::string("engine launch: ") + hipGetErrorString(e));
    if (a.trace) {
        std::vector<uint64_t> h(trace_n);
        HIP_TRY(c, hipMemcpyAsync(h.data(), a.trace, trace_n * sizeof(uint64_t), hipMemcpyDeviceToHost, c->stream));
        HIP_TRY(c, hipStreamSynchronize(c->stream));
        if (FILE *f = std::fopen(trace_path, "ab")) {
            const int32_t hdr[2] = {a.nops, P.grid};
            std::fwrite(hdr, sizeof(hdr), 1, f);
            for (const EngOp &op : P.ops) std::fwrite(&op.kind, sizeof(int32_t), 1, f);
            for (const EngOp &op : P.ops) std::fwrite(&op.ntasks, sizeof(int32_t), 1, f);
            std::fwrite(h.data(), sizeof(uint64_t), trace_n, f);
            std::fclose(f);
        }
    }
    return QTTS_OK;
}

qtts_status eng_status_check(qtts_ctx *c, const char *what) {
    int st[2] = {0, 0};
    HIP_TRY(c, hipMemcpy(st, c->eng_done, sizeof(st), hipMemcpyDeviceToHost));
    if (st[1] == QTTS_ENAN) return fail(c, QTTS_ENAN, std::string(what) + ": NaN logits (the reference panics)");
    if (st[1] != 0) return fail(c, (qtts_status)st[1], std::string(what) + ": engine wait timed out");
    return QTTS_OK;
}

// Talker attention splits of ~64 positions of the cache capacity: a split's
// K/V rows (1 KB per position) stream into one CU at ~25-30 GB/s, so short
// splits keep the attention step near its hand-off latency at long contexts,
// while fewer splits shorten the combine (with 512-thread blocks, 64 measured
// ahead of 48 and 96 on the 500-code loop's caches).
// Past 32 splits (8,192 rows), as many as keep a split within the attention
// step's 256-position score buffer, up to kEngMaxSplit (32,768 rows; the
// attention then runs several tasks per block).
int eng_talker_nsplit(int cap) {
    int n = (cap + 63) / 64;
    if (n < 1) n = 1;
    if (n > 32) n = 32;
    const int fit = (cap + 255) / 256;
    if (n < fit) n = fit;
    return n > kEngMaxSplit ? kEngMaxSplit : n;
}
bool eng_talker_fits(int cap) { return (cap + 255) / 256 <= kEngMaxSplit; }

// Passes 2.. of generate_acoustic_codes (src/code_predictor.rs:218-273)
// project the previous code's embedding, emb[g-1][code], to the predictor's
// width.  That projection depends only on the code, so it is applied ahead of
// time to every code of emb[0 .. groups-2] (in_proj(row) + bias), and a pass
// reads its input row by code.  The table is made by the matrix-core GEMM
// when the weight allows it (the same f32 products, summed in another order,
// so a row may differ from the step's GEMV by rounding), else by the GEMV.
// QTTS_PREDICTOR_TABLE=0 keeps the projection as a step.
qtts_status make_predictor_tables(qtts_predictor *p) {
    if (p->tab_state != 0) return QTTS_OK;
    p->tab_state = -1;
    const char *e = std::getenv("QTTS_PREDICTOR_TABLE");
    if ((e && std::strcmp(e, "0") == 0) || p->identity_proj || p->groups < 2) return QTTS_OK;
    qtts_ctx *c = p->ctx;
    const int rows = p->emb[0].K, th = p->talker_hidden, H = p->st.hidden, nt = p->groups - 1;
    for (int g = 0; g < nt; g++)
        if (p->emb[g].K != rows || p->emb[g].N != th) return QTTS_OK;
    float *tab = nullptr;
    QTTS_TRY(p->own.alloc(c, &tab, (size_t)nt * rows * H));
    Owner tmp;  // freed on return (hipFree waits for the stream's work)
    float *x = nullptr;
    uint32_t *ids = nullptr;
    QTTS_TRY(tmp.alloc(c, &x, (size_t)rows * th));
    QTTS_TRY(tmp.alloc(c, &ids, (size_t)rows));
    std::vector<uint32_t> h((size_t)rows);
    for (int i = 0; i < rows; i++) h[(size_t)i] = (uint32_t)i;
    HIP_TRY(c, hipMemcpyAsync(ids, h.data(), sizeof(uint32_t) * rows, hipMemcpyHostToDevice, c->stream));
    // Matrix-core copies of the two weights (one GEMM per table), else GEMV
    // launches of kMaxM rows.
    const Stack &st = p->st;
    const int nqkv = st.nq * st.hd + 2 * st.nkv * st.hd;
    DevQ4Mfma m_in{}, m_qkv{};
    bool ok_in = false, ok_qkv = false;
    void *mem = nullptr;
    if (rows >= kMfmaMinRows) {
        QTTS_TRY(make_mfma_copy(c, p->in_proj, &mem, &m_in, &ok_in));
        if (mem) tmp.ptrs.push_back(mem);
        QTTS_TRY(make_mfma_copy(c, st.L[0].qkv, &mem, &m_qkv, &ok_qkv));
        if (mem) tmp.ptrs.push_back(mem);
    }
    float *qkv = nullptr;
    QTTS_TRY(p->own.alloc(c, &qkv, (size_t)nt * rows * nqkv));
    for (int g = 0; g < nt; g++) {
        float *tg = tab + (size_t)g * rows * H, *qg = qkv + (size_t)g * rows * nqkv;
        launch_embed_rows(c->stream, p->emb[g], ids, 1, rows, x, th);
        QTTS_TRY(check_launch(c, "k_embed_rows"));
        if (ok_in) {
            QTTS_TRY(run_gemm_mfma(c, m_in, x, rows, th, MFMA_ROWS_PLAIN, nullptr, tg, H, p->bias, false));
        } else {
            for (int r0 = 0; r0 < rows; r0 += kMaxM) {
                GemvParams q = gemv_base(c, p->in_proj, rows - r0 < kMaxM ? rows - r0 : kMaxM);
                q.prologue = PRO_PLAIN;
                q.x = x + (size_t)r0 * th;
                q.ldx = th;
                q.epilogue = EPI_STORE;
                q.y = tg + (size_t)r0 * H;
                q.ldy = H;
                q.bias = p->bias;
                QTTS_TRY(run_gemv(c, q));
            }
        }
        // layer 0's q|k|v projection of every row, RMSNorm first (the first
        // step of such a pass, also a function of the code alone)
        if (ok_qkv) {
            QTTS_TRY(run_gemm_mfma(c, m_qkv, tg, rows, H, MFMA_ROWS_RMSNORM, st.L[0].in_g, qg, nqkv, nullptr, false));
        } else {
            for (int r0 = 0; r0 < rows; r0 += kMaxM) {
                GemvParams q = gemv_base(c, st.L[0].qkv, rows - r0 < kMaxM ? rows - r0 : kMaxM);
                q.prologue = PRO_RMSNORM;
                q.x = tg + (size_t)r0 * H;
                q.ldx = H;
                q.gamma = st.L[0].in_g;
                q.epilogue = EPI_STORE;
                q.y = qg + (size_t)r0 * nqkv;
                q.ldy = nqkv;
                QTTS_TRY(run_gemv(c, q));
            }
        }
    }
    QTTS_TRY(sync(c));
    p->tab = tab;
    p->qkv_tab = qkv;
    p->tab_rows = rows;
    p->tab_state = 1;
    return QTTS_OK;
}

qtts_status build_predictor_passes(EngProgram &P, qtts_predictor *p, qtts_kv *kv, const EngInput &row0,
                                   const EngInput &row1, TvRef *codes) {
    const Stack &st = p->st;
    QTTS_TRY(make_predictor_tables(p));
    // Every pass repeats the first pass's rotations, so a layer's attention
    // runs on the same blocks in all passes (its K/V rows stay in their LDS).
    std::vector<int> rots;
    P.rot_record = &rots;
    const size_t first = P.ops.size();
    GemvSpec ip;
    ip.M = 2;
    ip.in[0] = row0;
    ip.in[1] = row1;
    ip.bias = p->bias;
    TvRef x = add_gemv(P, p->in_proj, ip);
    for (int l = 0; l < st.layers; l++) x = add_layer(P, st, l, kv, 2, x, false, 0, 0, 1);
    GemvSpec hd;
    hd.norm = true;
    hd.gamma = st.final_g;
    hd.in[0] = in_tv(x, 1);
    if (p->tab_state == 1 && P.ops.size() > first + 2 && P.ops[first + 2].kind == EOP_ATTN) {
        // Passes 2-15 run the head right before the next pass's layer-0
        // attention: its blocks go where the one-row passes leave them free
        // of that attention's blocks and of the last down step's.
        const EngOp &dn = P.ops.back(), &a0 = P.ops[first + 2];
        const int nd = dn.ntasks / (dn.kind == EOP_GEMV && dn.gemv.M > 1 ? dn.gemv.M : 1);
        const int nh = p->heads[0].N / 32;
        auto in_range = [&](int b, int r, int n) { return ((b - r) % P.grid + P.grid) % P.grid < n; };
        for (int k = 0; k < P.grid; k++) {
            const int r = (dn.rot + nd + k) % P.grid;
            bool ok = nh + nd + a0.ntasks <= P.grid;
            for (int i = 0; ok && i < nh; i++) {
                const int b = (r + i) % P.grid;
                ok = !in_range(b, dn.rot, nd) && !in_range(b, a0.rot, a0.ntasks);
            }
            if (ok) {
                P.rot_next = r;
                break;
            }
        }
    }
    TvRef lg = add_gemv(P, p->heads[0], hd);
    const bool tab = p->tab_state == 1;
    // With the q|k|v table the later passes start at layer 0's attention,
    // which must keep its rows in LDS (as this pass's does).
    const bool qtab = tab && P.ops.size() > first + 2 && P.ops[first + 2].kind == EOP_ATTN &&
                      P.ops[first + 2].attn.lds_kv == 1;
    if (tab && P.ops.size() > first + 2) {
        // The argmax step's block runs no task of the next pass's first
        // step (the one-row version of this pass's QKV step, or the
        // attention), which computes the same argmax itself.
        const EngOp &q = P.ops[first + (qtab ? 2 : 1)];
        const int n = q.ntasks / (q.kind == EOP_GEMV && q.gemv.M > 1 ? q.gemv.M : 1);
        if (n < P.grid) P.rot_next = (q.rot + n) % P.grid;
    }
    codes[0] = add_argmax(P, lg, p->vocab, 1);
    P.rot_record = nullptr;
    for (int g = 1; g < p->groups; g++) {
        P.rot_plan = &rots;
        P.plan_pos = 0;
        if (tab) {
            // The input projection of the previous code is a table row: the
            // first layer reads it at the argmax of the previous logits
            // (the argmax step still files and publishes the code).
            P.plan_pos = qtab ? 2 : 1;
            TabIn ti;
            ti.logits = lg;
            ti.n = p->vocab;
            ti.table = p->tab + (size_t)(g - 1) * p->tab_rows * st.hidden;
            ti.rows = p->tab_rows;
            ti.code = codes[g - 1];
            if (qtab) ti.qkv_table = p->qkv_tab + (size_t)(g - 1) * p->tab_rows * (st.nq * st.hd + 2 * st.nkv * st.hd);
            x = add_layer(P, st, 0, kv, 1, TvRef{}, false, g + 1, g + 1, 1, &ti);
        } else {
            GemvSpec e;
            e.in[0] = in_embed(p->emb[g - 1], codes[g - 1]);
            e.bias = p->bias;
            x = add_gemv(P, p->in_proj, e);
            x = add_layer(P, st, 0, kv, 1, x, false, g + 1, g + 1, 1);
        }
        for (int l = 1; l < st.layers; l++) x = add_layer(P, st, l, kv, 1, x, false, g + 1, g + 1, 1);
        hd.in[0] = in_tv(x, 0);
        lg = add_gemv(P, p->heads[g], hd);
        codes[g] = add_argmax(P, lg, p->vocab, g + 1);
        P.rot_plan = nullptr;
    }
    return QTTS_OK;
}

qtts_status build_talker_layers_and_head(EngProgram &P, qtts_talker *t, qtts_kv *kv, TvRef x, int nsplit) {
    for (int l = 0; l < t->st.layers; l++) x = add_layer(P, t->st, l, kv, 1, x, true, 0, 0, nsplit);
    GemvSpec h;
    h.norm = true;
    h.gamma = t->st.final_g;
    h.in[0] = in_tv(x, 0);
    h.kc = 1;
    h.out_plain = t->out + t->st.hidden;  // logits, read by the next frame's sampler
    h.norm_plain = t->out;                // normed hidden, read by the next predictor frame
    add_gemv(P, t->head, h);
    return QTTS_OK;
}

}  // namespace

// ===========================================================================
// C-ABI
// ===========================================================================
extern "C" {

const char *qtts_version(void) { return "qtts-mi355x 0.1.0 (gfx950)"; }

qtts_status qtts_ctx_create(int32_t device, qtts_ctx **out) {
    if (!out) return QTTS_EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return QTTS_EDEVICE;
    if (device < 0 || device >= n) return QTTS_EINVAL;
    qtts_ctx *c = new qtts_ctx();
    c->device = device;
    auto bad = [&](hipError_t e) {
        if (e == hipSuccess) return false;
        qtts_ctx_destroy(c);
        return true;
    };
    if (bad(hipSetDevice(device))) return QTTS_EDEVICE;
    if (bad(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking))) return QTTS_EDEVICE;
    if (bad(hipMalloc(&c->partial, kPartialFloats * sizeof(float)))) return QTTS_ENOMEM;
    if (bad(hipMalloc(&c->counters, kCounters * sizeof(unsigned)))) return QTTS_ENOMEM;
    if (bad(hipMalloc(&c->attn_part, kAttnPartFloats * sizeof(float)))) return QTTS_ENOMEM;
    if (bad(hipMalloc(&c->attn_counters, kAttnCounters * sizeof(unsigned)))) return QTTS_ENOMEM;
    if (bad(hipMalloc(&c->d_small, 256))) return QTTS_ENOMEM;
    if (bad(hipMemset(c->counters, 0, kCounters * sizeof(unsigned)))) return QTTS_EDEVICE;
    if (bad(hipMemset(c->attn_counters, 0, kAttnCounters * sizeof(unsigned)))) return QTTS_EDEVICE;
    if (bad(static_scratch_setup(device))) return QTTS_EDEVICE;
    if (bad(hipDeviceSynchronize())) return QTTS_EDEVICE;
    *out = c;
    return QTTS_OK;
}

void qtts_ctx_destroy(qtts_ctx *c) {
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    ctx_release(c);
}

const char *qtts_last_error(const qtts_ctx *c) { return c ? c->err.c_str() : "null context"; }

void *qtts_ctx_stream(qtts_ctx *c) { return c ? (void *)c->stream : nullptr; }

qtts_status qtts_ctx_synchronize(qtts_ctx *c) {
    if (!c) return QTTS_EINVAL;
    return sync(c);
}

// ---------------------------------------------------------------------------
qtts_status qtts_q4_upload(qtts_ctx *c, const qtts_q4_view *v, qtts_q4 **out) {
    if (!c || !v || !out) return QTTS_EINVAL;
    *out = nullptr;
    if (!v->packed || !v->scales) return fail(c, QTTS_EINVAL, "null weight arrays");
    if (v->k <= 0 || v->n <= 0 || v->n % 32 != 0) return fail(c, QTTS_ESHAPE, "Q4 weight needs n % 32 == 0");
    qtts_q4 *w = new qtts_q4();
    w->ctx = ctx_retain(c);
    w->bytes = (size_t)v->k * v->n / 2 + (size_t)v->k * (v->n / 32) * 2;
    if (hipMalloc(&w->mem, w->bytes) != hipSuccess) {
        delete w;
        return fail(c, QTTS_ENOMEM, "hipMalloc weight");
    }
    w->d.wq = reinterpret_cast<const uint4 *>(w->mem);
    w->d.ws = reinterpret_cast<const uint16_t *>((uint8_t *)w->mem + (size_t)v->k * v->n / 2);
    w->d.K = v->k;
    w->d.N = v->n;
    qtts_status s = upload_part(c, v, w->d, 0);
    if (s != QTTS_OK) {
        qtts_q4_free(w);
        return s;
    }
    *out = w;
    return QTTS_OK;
}

void qtts_q4_free(qtts_q4 *w) {
    if (!w) return;
    qtts_ctx *c = w->ctx;
    if (c && c->stream) (void)hipStreamSynchronize(c->stream);
    (void)hipFree(w->mem);
    (void)hipFree(w->mfma_mem);
    delete w;
    if (c) ctx_release(c);
}

size_t qtts_q4_bytes(const qtts_q4 *w) { return w ? w->bytes : 0; }

qtts_status qtts_gemm_device(qtts_ctx *c, const qtts_q4 *w, const float *d_x, int32_t seq_len, float *d_out) {
    if (!c || !w || !d_x || !d_out) return QTTS_EINVAL;
    if (seq_len < 1) return fail(c, QTTS_EINVAL, "seq_len < 1");
    if (seq_len >= kMfmaMinRows && ((uintptr_t)d_x & 15) == 0) {
        qtts_q4 *mw = const_cast<qtts_q4 *>(w);
        if (mw->mfma_state == 0) {
            bool ok = false;
            QTTS_TRY(make_mfma_copy(c, w->d, &mw->mfma_mem, &mw->m, &ok));
            mw->mfma_state = ok ? 1 : -1;
        }
        if (mw->mfma_state == 1)
            return run_gemm_mfma(c, w->m, d_x, seq_len, w->d.K, MFMA_ROWS_PLAIN, nullptr, d_out, w->d.N, nullptr,
                                 false);
    }
    for (int r0 = 0; r0 < seq_len; r0 += kMaxM) {
        const int M = seq_len - r0 < kMaxM ? seq_len - r0 : kMaxM;
        GemvParams p = gemv_base(c, w->d, M);
        p.prologue = PRO_PLAIN;
        p.x = d_x + (size_t)r0 * w->d.K;
        p.ldx = w->d.K;
        p.epilogue = EPI_STORE;
        p.y = d_out + (size_t)r0 * w->d.N;
        p.ldy = w->d.N;
        QTTS_TRY(run_gemv(c, p));
    }
    return QTTS_OK;
}

qtts_status qtts_gemv_device(qtts_ctx *c, const qtts_q4 *w, const float *d_x, float *d_out) {
    return qtts_gemm_device(c, w, d_x, 1, d_out);
}

qtts_status qtts_gemv_device_static(const qtts_q4 *w, const float *d_x, int32_t rows, float *d_out, void *stream) {
    if (!w || !d_x || !d_out) return QTTS_EINVAL;
    qtts_ctx *c = w->ctx;
    if (rows < 1 || rows > kMaxM) return fail(c, QTTS_ERANGE, "gemv_device_static: rows must be 1..4");
    if (w->d.K > kStaticMaxK || w->d.N > kStaticMaxN)
        return fail(c, QTTS_ERANGE, "gemv_device_static: K above 8192 or N above 16384");
    float *scr = static_cast<float *>(static_scratch(c->device));
    if (!scr) return fail(c, QTTS_ESTATE, "gemv_device_static: no scratch on this device");
    GemvParams p{};
    p.w = w->d;
    p.M = rows;
    plan_gemv(w->d.K, w->d.N, rows, &p.kc, &p.rpt);
    if (p.kc > kStaticMaxChunks) return fail(c, QTTS_ERANGE, "gemv_device_static: too many K chunks");
    p.prologue = PRO_PLAIN;
    p.x = d_x;
    p.ldx = w->d.K;
    p.epilogue = EPI_STORE;
    p.y = d_out;
    p.ldy = w->d.N;
    p.partial = scr;
    p.counters = reinterpret_cast<unsigned *>(scr + kStaticPartialFloats);
    launch_gemv(stream ? static_cast<hipStream_t>(stream) : c->stream, p);
    return check_launch(c, "k_gemv");
}

qtts_status qtts_gemm(qtts_ctx *c, const qtts_q4 *w, const float *x, int32_t seq_len, float *out) {
    if (!c || !w || !x || !out) return QTTS_EINVAL;
    if (seq_len < 1) return fail(c, QTTS_EINVAL, "seq_len < 1");
    const size_t nin = (size_t)seq_len * w->d.K, nout = (size_t)seq_len * w->d.N;
    QTTS_TRY(ensure_staging(c, nin, nout));
    HIP_TRY(c, hipMemcpyAsync(c->d_in, x, nin * sizeof(float), hipMemcpyHostToDevice, c->stream));
    QTTS_TRY(qtts_gemm_device(c, w, c->d_in, seq_len, c->d_out));
    HIP_TRY(c, hipMemcpyAsync(out, c->d_out, nout * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

qtts_status qtts_gemv(qtts_ctx *c, const qtts_q4 *w, const float *input, float *output) {
    return qtts_gemm(c, w, input, 1, output);
}

qtts_status qtts_embed_lookup(qtts_ctx *c, const qtts_q4 *w, int32_t token_id, float *out) {
    if (!c || !w || !out) return QTTS_EINVAL;
    if (token_id < 0 || token_id >= w->d.K) return fail(c, QTTS_ERANGE, "token id out of range");
    QTTS_TRY(ensure_staging(c, 0, (size_t)w->d.N));
    const uint32_t tok = (uint32_t)token_id;
    HIP_TRY(c, hipMemcpyAsync(c->d_small, &tok, 4, hipMemcpyHostToDevice, c->stream));
    launch_embed_row(c->stream, w->d, c->d_small, c->d_out, nullptr);
    QTTS_TRY(check_launch(c, "k_embed_row"));
    HIP_TRY(c, hipMemcpyAsync(out, c->d_out, (size_t)w->d.N * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

// ---------------------------------------------------------------------------
qtts_status qtts_kv_create(qtts_ctx *c, int32_t num_layers, int32_t num_kv_heads, int32_t head_dim, int32_t capacity,
                           qtts_kv **out) {
    if (!c || !out) return QTTS_EINVAL;
    *out = nullptr;
    if (num_layers <= 0 || num_kv_heads <= 0 || head_dim <= 0 || capacity <= 0)
        return fail(c, QTTS_EINVAL, "kv dimensions must be positive");
    qtts_kv *kv = new qtts_kv();
    kv->ctx = ctx_retain(c);
    kv->layers = num_layers;
    kv->kvh = num_kv_heads;
    kv->hd = head_dim;
    kv->cap = capacity;
    const size_t bytes = (size_t)num_layers * num_kv_heads * capacity * head_dim * sizeof(float);
    if (hipMalloc(&kv->k, bytes) != hipSuccess || hipMalloc(&kv->v, bytes) != hipSuccess) {
        qtts_kv_free(kv);
        return fail(c, QTTS_ENOMEM, "hipMalloc kv cache");
    }
    if (hipMemset(kv->k, 0, bytes) != hipSuccess || hipMemset(kv->v, 0, bytes) != hipSuccess) {
        qtts_kv_free(kv);
        return fail(c, QTTS_EDEVICE, "hipMemset kv cache");
    }
    *out = kv;
    return QTTS_OK;
}

void qtts_kv_free(qtts_kv *kv) {
    if (!kv) return;
    qtts_ctx *c = kv->ctx;
    if (c && c->stream) (void)hipStreamSynchronize(c->stream);
    (void)hipFree(kv->k);
    (void)hipFree(kv->v);
    delete kv;
    if (c) ctx_release(c);
}

int32_t qtts_kv_len(const qtts_kv *kv) { return kv ? kv->len : -1; }

qtts_status qtts_kv_clear(qtts_kv *kv) {
    if (!kv) return QTTS_EINVAL;
    kv->len = 0;
    return QTTS_OK;
}

qtts_status qtts_kv_load(qtts_kv *kv, const float *k, const float *v, int32_t len) {
    if (!kv || !k || !v) return QTTS_EINVAL;
    qtts_ctx *c = kv->ctx;
    if (len < 0 || len > kv->cap) return fail(c, QTTS_ERANGE, "kv_load: len exceeds capacity");
    const size_t row = (size_t)kv->kvh * kv->hd;
    std::vector<float> tk((size_t)kv->kvh * kv->cap * kv->hd), tv(tk.size());
    for (int l = 0; l < kv->layers; l++) {
        const float *sk = k + (size_t)l * len * row, *sv = v + (size_t)l * len * row;
        for (int t = 0; t < len; t++)
            for (int hh = 0; hh < kv->kvh; hh++) {
                std::memcpy(&tk[((size_t)hh * kv->cap + t) * kv->hd], sk + t * row + (size_t)hh * kv->hd,
                            sizeof(float) * kv->hd);
                std::memcpy(&tv[((size_t)hh * kv->cap + t) * kv->hd], sv + t * row + (size_t)hh * kv->hd,
                            sizeof(float) * kv->hd);
            }
        HIP_TRY(c, hipMemcpy(kv->layer_k(l), tk.data(), tk.size() * sizeof(float), hipMemcpyHostToDevice));
        HIP_TRY(c, hipMemcpy(kv->layer_v(l), tv.data(), tv.size() * sizeof(float), hipMemcpyHostToDevice));
    }
    kv->len = len;
    return QTTS_OK;
}

qtts_status qtts_kv_store(const qtts_kv *kv, float *k, float *v) {
    if (!kv || !k || !v) return QTTS_EINVAL;
    qtts_ctx *c = kv->ctx;
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    const size_t row = (size_t)kv->kvh * kv->hd;
    std::vector<float> tk((size_t)kv->kvh * kv->cap * kv->hd), tv(tk.size());
    for (int l = 0; l < kv->layers; l++) {
        HIP_TRY(c, hipMemcpy(tk.data(), kv->layer_k(l), tk.size() * sizeof(float), hipMemcpyDeviceToHost));
        HIP_TRY(c, hipMemcpy(tv.data(), kv->layer_v(l), tv.size() * sizeof(float), hipMemcpyDeviceToHost));
        float *dk = k + (size_t)l * kv->len * row, *dv = v + (size_t)l * kv->len * row;
        for (int t = 0; t < kv->len; t++)
            for (int hh = 0; hh < kv->kvh; hh++) {
                std::memcpy(dk + t * row + (size_t)hh * kv->hd, &tk[((size_t)hh * kv->cap + t) * kv->hd],
                            sizeof(float) * kv->hd);
                std::memcpy(dv + t * row + (size_t)hh * kv->hd, &tv[((size_t)hh * kv->cap + t) * kv->hd],
                            sizeof(float) * kv->hd);
            }
    }
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
qtts_status qtts_talker_upload(qtts_ctx *c, const qtts_talker_view *v, qtts_talker **out) {
    if (!c || !v || !out) return QTTS_EINVAL;
    *out = nullptr;
    qtts_talker *t = new qtts_talker();
    t->ctx = ctx_retain(c);
    auto bail = [&](qtts_status s) {
        delete t;
        return s;
    };
    qtts_status s =
        upload_stack(c, t->own, v->num_layers, v->layers, v->hidden_size, v->num_heads, v->num_kv_heads, v->head_dim, &t->st);
    if (s != QTTS_OK) return bail(s);
    const int hidden = v->hidden_size;
    t->vocab = v->codec_head.n;
    t->max_pos = v->max_position;
    if ((s = check_view(c, &v->codec_head, hidden, t->vocab, "codec_head")) != QTTS_OK) return bail(s);
    if ((s = check_view(c, &v->codec_embedding, v->codec_embedding.k, hidden, "codec_embedding")) != QTTS_OK)
        return bail(s);
    if (v->max_position <= 0) return bail(fail(c, QTTS_EINVAL, "max_position must be positive"));
    if ((s = alloc_q4(c, t->own, hidden, t->vocab, &t->head)) != QTTS_OK) return bail(s);
    if ((s = upload_part(c, &v->codec_head, t->head, 0)) != QTTS_OK) return bail(s);
    if ((s = alloc_q4(c, t->own, v->codec_embedding.k, hidden, &t->emb)) != QTTS_OK) return bail(s);
    if ((s = upload_part(c, &v->codec_embedding, t->emb, 0)) != QTTS_OK) return bail(s);
    if ((s = upload_array(c, t->own, v->final_norm_gamma, (size_t)hidden, &t->st.final_g, "final_norm_gamma")) !=
        QTTS_OK)
        return bail(s);
    if ((s = upload_rope(c, t->own, v->head_dim, v->max_position, v->rope_theta, v->rope_cos, v->rope_sin, &t->st)) != QTTS_OK) return bail(s);
    t->st.rope_skip_oob = 0;
    const int qd = t->st.nq * t->st.hd;
    if ((s = t->own.alloc(c, &t->x, (size_t)hidden)) != QTTS_OK) return bail(s);
    if ((s = t->own.alloc(c, &t->q, (size_t)qd)) != QTTS_OK) return bail(s);
    if ((s = t->own.alloc(c, &t->attn, (size_t)qd)) != QTTS_OK) return bail(s);
    if ((s = t->own.alloc(c, &t->h, (size_t)t->st.inter)) != QTTS_OK) return bail(s);
    if ((s = t->own.alloc(c, &t->out, (size_t)hidden + t->vocab)) != QTTS_OK) return bail(s);
    if ((s = t->own.alloc(c, &t->pad, (size_t)hidden)) != QTTS_OK) return bail(s);
    if ((s = t->own.alloc(c, &t->state, 1)) != QTTS_OK) return bail(s);
    if (hipMemset(t->state, 0, sizeof(LoopState)) != hipSuccess) return bail(fail(c, QTTS_EDEVICE, "memset"));
    *out = t;
    return QTTS_OK;
}

void qtts_talker_free(qtts_talker *t) {
    if (!t) return;
    qtts_ctx *c = t->ctx;
    if (c) (void)hipStreamSynchronize(c->stream);
    delete t;
    if (c) ctx_release(c);
}

namespace {

qtts_status check_kv(qtts_ctx *c, const Stack &st, const qtts_kv *kv) {
    if (!kv) return fail(c, QTTS_EINVAL, "null kv cache");
    if (kv->layers != st.layers || kv->kvh != st.nkv || kv->hd != st.hd)
        return fail(c, QTTS_ESHAPE, "kv cache shape does not match the model");
    return QTTS_OK;
}

qtts_status set_state(qtts_talker *t, int pos, int kvlen) {
    const int v[2] = {pos, kvlen};
    HIP_TRY(t->ctx, hipMemcpyAsync(t->state, v, sizeof(v), hipMemcpyHostToDevice, t->ctx->stream));
    return QTTS_OK;
}

// forward_with_embedding on device buffers: t->x holds the input embedding;
// hidden_out/logits_out receive [normed hidden] and [logits].
qtts_status enqueue_talker_step(qtts_talker *t, qtts_kv *kv, float *hidden_out, float *logits_out, const int *d_done,
                                int frame_step) {
    qtts_ctx *c = t->ctx;
    QTTS_TRY(enqueue_layers(c, t->st, kv, t->x, t->q, t->attn, t->h, 1, &t->state->pos, 0, &t->state->kvlen, 0,
                            t->nsplit, d_done));
    GemvParams p = gemv_base(c, t->head, 1);
    p.prologue = PRO_RMSNORM;
    p.x = t->x;
    p.ldx = t->st.hidden;
    p.gamma = t->st.final_g;
    p.norm_out = hidden_out;
    p.ldn = t->st.hidden;
    p.epilogue = EPI_STORE;
    p.y = logits_out;
    p.ldy = t->vocab;
    p.d_done = d_done;
    QTTS_TRY(run_gemv(c, p));
    launch_advance(c->stream, t->state, frame_step);
    return check_launch(c, "k_advance");
}

}  // namespace

namespace {

qtts_status talker_step_check(qtts_talker *t, qtts_kv *kv, int32_t position) {
    qtts_ctx *c = t->ctx;
    QTTS_TRY(check_kv(c, t->st, kv));
    if (position < 0 || position >= t->max_pos) return fail(c, QTTS_ERANGE, "position beyond the RoPE table");
    if (kv->len + 1 > kv->cap) return fail(c, QTTS_ERANGE, "kv cache full");
    return QTTS_OK;
}

// forward_with_embedding (src/talker.rs:263-360) of the embedding already in
// t->x (enqueued before this call); [hidden ++ logits] to the host `out`
// (out_n floats of it).
qtts_status talker_step_x(qtts_talker *t, qtts_kv *kv, int32_t position, float *out, int out_n) {
    qtts_ctx *c = t->ctx;
    const int hidden = t->st.hidden;
    if (engine_enabled() && eng_talker_fits(kv->cap)) {
        QTTS_TRY(eng_init(c));
        if (!t->step_prog || t->step_kv != kv->serial) {
            t->step_prog.reset(new EngProgram());
            const int nsplit = eng_talker_nsplit(kv->cap);
            QTTS_TRY(eng_build(c, *t->step_prog, [&](EngProgram &P) {
                TvRef x = add_embsum(P, 2, nullptr, nullptr, nullptr, 0, TvRef{}, nullptr, 0, t->x, hidden);
                return build_talker_layers_and_head(P, t, kv, x, nsplit);
            }));
            t->step_kv = kv->serial;
        }
        if (!t->step_prog->unsupported) {
            QTTS_TRY(eng_reset(c, position, kv->len, 0));
            QTTS_TRY(eng_launch(c, *t->step_prog, 0, c->d_small, 1));
            HIP_TRY(c, hipMemcpyAsync(out, t->out, sizeof(float) * out_n, hipMemcpyDeviceToHost, c->stream));
            QTTS_TRY(sync(c));
            QTTS_TRY(eng_status_check(c, "forward_with_embedding"));
            kv->len += 1;
            return QTTS_OK;
        }
    }
    t->nsplit = attn_nsplit_row(kv->cap);
    QTTS_TRY(set_state(t, position, kv->len));
    QTTS_TRY(enqueue_talker_step(t, kv, t->out, t->out + hidden, nullptr, 0));
    HIP_TRY(c, hipMemcpyAsync(out, t->out, sizeof(float) * out_n, hipMemcpyDeviceToHost, c->stream));
    QTTS_TRY(sync(c));
    kv->len += 1;
    return QTTS_OK;
}

}  // namespace

qtts_status qtts_forward_with_embedding(qtts_talker *t, const float *embedding, qtts_kv *kv, int32_t position,
                                        float *out) {
    if (!t || !embedding || !out) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    QTTS_TRY(talker_step_check(t, kv, position));
    HIP_TRY(c, hipMemcpyAsync(t->x, embedding, sizeof(float) * t->st.hidden, hipMemcpyHostToDevice, c->stream));
    return talker_step_x(t, kv, position, out, t->st.hidden + t->vocab);
}

// Prefill layers on the GEMV path: row chunks of up to kMaxM tokens, in
// order, layer by layer (a chunk's causal attention reads the K/V rows that
// earlier chunks appended).
static qtts_status prefill_layers_rows(qtts_talker *t, qtts_kv *kv, int seq_len) {
    qtts_ctx *c = t->ctx;
    const Stack &st = t->st;
    const int hidden = st.hidden, qd = st.nq * st.hd;
    Stack one = st;
    for (int l = 0; l < st.layers; l++) {
        one.layers = 1;
        one.L.assign(1, st.L[l]);
        qtts_kv layer_kv = *kv;
        layer_kv.layers = 1;
        layer_kv.k = kv->layer_k(l);
        layer_kv.v = kv->layer_v(l);
        for (int r0 = 0; r0 < seq_len; r0 += kMaxM) {
            const int M = seq_len - r0 < kMaxM ? seq_len - r0 : kMaxM;
            QTTS_TRY(enqueue_layers(c, one, &layer_kv, t->xp + (size_t)r0 * hidden, t->qp + (size_t)r0 * qd,
                                    t->ap + (size_t)r0 * qd, t->hp + (size_t)r0 * st.inter, M, nullptr, r0, nullptr,
                                    r0, t->nsplit, nullptr));
        }
    }
    return QTTS_OK;
}

// The MFMA operand copies of every layer weight; t->mfma_state -1 (and no
// copies kept) when any weight cannot take the matrix-core path.
static qtts_status make_talker_mfma(qtts_talker *t) {
    qtts_ctx *c = t->ctx;
    std::vector<DevQ4Mfma> copies;
    std::vector<void *> mems;
    bool all = true;
    for (const DevLayer &Ly : t->st.L) {
        for (const DevQ4 *w : {&Ly.qkv, &Ly.o, &Ly.gu, &Ly.down}) {
            DevQ4Mfma m{};
            void *mem = nullptr;
            bool ok = false;
            const qtts_status s = make_mfma_copy(c, *w, &mem, &m, &ok);
            if (s != QTTS_OK || !ok) {
                for (void *p : mems) (void)hipFree(p);
                if (s != QTTS_OK) return s;
                all = false;
                break;
            }
            mems.push_back(mem);
            copies.push_back(m);
        }
        if (!all) break;
    }
    if (!all) {
        t->mfma_state = -1;
        return QTTS_OK;
    }
    for (void *p : mems) t->own.ptrs.push_back(p);
    t->mfma = std::move(copies);
    t->mfma_state = 1;
    return QTTS_OK;
}

// Prefill layers on the matrix cores (csrc/mfma.hip), all rows at once per
// layer: QKV (RMSNorm prologue) -> QK-norm, RoPE, KV append -> causal
// attention (row r sees positions 0..r) -> O (+residual) -> gate|up (RMSNorm
// prologue) -> down (SiLU*up prologue, +residual); src/talker.rs:364-462.
static qtts_status prefill_layers_mfma(qtts_talker *t, qtts_kv *kv, int seq_len) {
    qtts_ctx *c = t->ctx;
    const Stack &st = t->st;
    const int hidden = st.hidden, qd = st.nq * st.hd, nqkv = qd + 2 * st.nkv * st.hd;
    // one attention split per kAttnMaxChunk positions of the prefill (the
    // decode-sized split count would give thousands of tiny blocks)
    const int nsplit = attn_nsplit(seq_len, 1);
    int attn_rows = (int)(kAttnPartFloats / ((size_t)st.nq * nsplit * (st.hd + 2)));
    if (attn_rows > kAttnCounters / st.nkv) attn_rows = kAttnCounters / st.nkv;
    if (attn_rows < 1) return fail(c, QTTS_ESHAPE, "attention split buffer too small");
    for (int l = 0; l < st.layers; l++) {
        const DevLayer &Ly = st.L[l];
        const DevQ4Mfma *W = &t->mfma[(size_t)4 * l];
        float *kc = kv->layer_k(l), *vc = kv->layer_v(l);
        QTTS_TRY(run_gemm_mfma(c, W[0], t->xp, seq_len, hidden, MFMA_ROWS_RMSNORM, Ly.in_g, t->rawp, nqkv, nullptr,
                               false));
        QkvRowsParams q{};
        q.raw = t->rawp;
        q.ldr = nqkv;
        q.M = seq_len;
        q.n_q_heads = st.nq;
        q.n_kv_heads = st.nkv;
        q.head_dim = st.hd;
        q.q_norm = Ly.q_norm;
        q.k_norm = Ly.k_norm;
        q.rope_cos = st.rope_cos;
        q.rope_sin = st.rope_sin;
        q.rope_rows = st.rope_rows;
        q.rope_skip_oob = st.rope_skip_oob;
        q.q = t->qp;
        q.ldq = qd;
        q.kcache = kc;
        q.vcache = vc;
        q.kv_cap = kv->cap;
        launch_qkv_rows(c->stream, q);
        QTTS_TRY(check_launch(c, "k_qkv_rows"));
        for (int r0 = 0; r0 < seq_len; r0 += attn_rows) {
            const int M = seq_len - r0 < attn_rows ? seq_len - r0 : attn_rows;
            AttnParams a{};
            a.q = t->qp + (size_t)r0 * qd;
            a.ldq = qd;
            a.kcache = kc;
            a.vcache = vc;
            a.kv_cap = kv->cap;
            a.nq = st.nq;
            a.nkv = st.nkv;
            a.hd = st.hd;
            a.kvlen_const = r0;
            a.nsplit = nsplit;
            a.scale = 1.0f / sqrtf((float)st.hd);  // src/talker.rs:305
            a.part = c->attn_part;
            a.counters = c->attn_counters;
            a.out = t->ap + (size_t)r0 * qd;
            a.ldo = qd;
            launch_attention(c->stream, a, M);
            QTTS_TRY(check_launch(c, "k_attn"));
        }
        QTTS_TRY(run_gemm_mfma(c, W[1], t->ap, seq_len, qd, MFMA_ROWS_PLAIN, nullptr, t->xp, hidden, nullptr, true));
        QTTS_TRY(run_gemm_mfma(c, W[2], t->xp, seq_len, hidden, MFMA_ROWS_RMSNORM, Ly.post_g, t->rawp, 2 * st.inter,
                               nullptr, false));
        QTTS_TRY(run_gemm_mfma(c, W[3], t->rawp, seq_len, 2 * st.inter, MFMA_ROWS_SWIGLU, nullptr, t->xp, hidden,
                               nullptr, true));
    }
    return QTTS_OK;
}

namespace {

qtts_status prefill_buffers(qtts_talker *t, int32_t seq_len);

// Checks a prefill of seq_len rows into kv and sizes the prefill work buffers.
qtts_status prefill_prepare(qtts_talker *t, int32_t seq_len, qtts_kv *kv) {
    qtts_ctx *c = t->ctx;
    QTTS_TRY(check_kv(c, t->st, kv));
    if (kv->len != 0) return fail(c, QTTS_ESTATE, "prefill needs an empty cache (src/talker.rs:405-408)");
    if (seq_len < 1) return fail(c, QTTS_EINVAL, "seq_len < 1");
    if (seq_len > kv->cap) return fail(c, QTTS_ERANGE, "prefill longer than the cache");
    if (seq_len > t->max_pos) return fail(c, QTTS_ERANGE, "prefill longer than the RoPE table");
    return prefill_buffers(t, seq_len);
}

// Sizes the prefill work buffers (t->xp and the per-row scratch) for seq_len rows.
qtts_status prefill_buffers(qtts_talker *t, int32_t seq_len) {
    qtts_ctx *c = t->ctx;
    const Stack &st = t->st;
    const int hidden = st.hidden, qd = st.nq * st.hd;
    if (seq_len > t->prefill_cap) {
        for (void *p : t->prefill_bufs) (void)hipFree(p);
        t->prefill_bufs.clear();
        t->prefill_cap = 0;
        HIP_TRY(c, hipMalloc(&t->xp, sizeof(float) * seq_len * hidden));
        t->prefill_bufs.push_back(t->xp);
        HIP_TRY(c, hipMalloc(&t->qp, sizeof(float) * seq_len * qd));
        t->prefill_bufs.push_back(t->qp);
        HIP_TRY(c, hipMalloc(&t->ap, sizeof(float) * seq_len * qd));
        t->prefill_bufs.push_back(t->ap);
        HIP_TRY(c, hipMalloc(&t->hp, sizeof(float) * seq_len * st.inter));
        t->prefill_bufs.push_back(t->hp);
        const size_t raw_cols = std::max((size_t)qd + 2 * st.nkv * st.hd, (size_t)2 * st.inter);
        HIP_TRY(c, hipMalloc(&t->rawp, sizeof(float) * seq_len * raw_cols));
        t->prefill_bufs.push_back(t->rawp);
        t->prefill_cap = seq_len;
    }
    return QTTS_OK;
}

// prefill_talker_raw (src/talker.rs:364-462) of the seq_len rows already in
// t->xp.  Leaves the final-normed last row in t->out[0, hidden) and its
// logits, apply_codec_head (src/talker.rs:627-629), in t->out + hidden.
qtts_status prefill_from_xp(qtts_talker *t, int32_t seq_len, qtts_kv *kv) {
    qtts_ctx *c = t->ctx;
    const Stack &st = t->st;
    const int hidden = st.hidden;
    t->nsplit = attn_nsplit_row(kv->cap);
    if (seq_len >= kMfmaMinRows && t->mfma_state == 0) QTTS_TRY(make_talker_mfma(t));
    if (seq_len >= kMfmaMinRows && t->mfma_state == 1) {
        QTTS_TRY(prefill_layers_mfma(t, kv, seq_len));
    } else {
        QTTS_TRY(prefill_layers_rows(t, kv, seq_len));
    }
    // final norm of the last row (src/talker.rs:460-461) via the head GEMV's
    // normalising prologue, which also forms the logits of that normed row
    GemvParams p = gemv_base(c, t->head, 1);
    p.prologue = PRO_RMSNORM;
    p.x = t->xp;
    p.ldx = hidden;
    p.norm_src_row0 = seq_len - 1;
    p.gamma = st.final_g;
    p.norm_out = t->out;
    p.ldn = hidden;
    p.epilogue = EPI_STORE;
    p.y = t->out + hidden;
    p.ldy = t->vocab;
    QTTS_TRY(run_gemv(c, p));
    kv->len = seq_len;
    return QTTS_OK;
}

}  // namespace

qtts_status qtts_prefill_talker_raw(qtts_talker *t, const float *x, int32_t seq_len, qtts_kv *kv, float *last_hidden) {
    if (!t || !x || !last_hidden) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    QTTS_TRY(prefill_prepare(t, seq_len, kv));
    HIP_TRY(c, hipMemcpyAsync(t->xp, x, sizeof(float) * seq_len * t->st.hidden, hipMemcpyHostToDevice, c->stream));
    qtts_status s = prefill_from_xp(t, seq_len, kv);
    if (s != QTTS_OK) {
        kv->len = 0;
        return s;
    }
    HIP_TRY(c, hipMemcpyAsync(last_hidden, t->out, sizeof(float) * t->st.hidden, hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

qtts_status qtts_apply_codec_head(qtts_talker *t, const float *hidden, float *logits) {
    if (!t || !hidden || !logits) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    HIP_TRY(c, hipMemcpyAsync(t->x, hidden, sizeof(float) * t->st.hidden, hipMemcpyHostToDevice, c->stream));
    GemvParams p = gemv_base(c, t->head, 1);
    p.prologue = PRO_PLAIN;
    p.x = t->x;
    p.ldx = t->st.hidden;
    p.epilogue = EPI_STORE;
    p.y = t->out + t->st.hidden;
    p.ldy = t->vocab;
    QTTS_TRY(run_gemv(c, p));
    HIP_TRY(c, hipMemcpyAsync(logits, t->out + t->st.hidden, sizeof(float) * t->vocab, hipMemcpyDeviceToHost,
                              c->stream));
    return sync(c);
}

qtts_status qtts_embed_codec_token(qtts_talker *t, uint32_t token_id, float *out) {
    if (!t || !out) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    if (token_id >= (uint32_t)t->emb.K) return fail(c, QTTS_ERANGE, "token id out of range");
    HIP_TRY(c, hipMemcpyAsync(c->d_small, &token_id, 4, hipMemcpyHostToDevice, c->stream));
    launch_embed_row(c->stream, t->emb, c->d_small, t->out, nullptr);
    QTTS_TRY(check_launch(c, "k_embed_row"));
    HIP_TRY(c, hipMemcpyAsync(out, t->out, sizeof(float) * t->st.hidden, hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

// ---------------------------------------------------------------------------
// Prompt assembly: embed_text_token (src/talker.rs:105-116),
// prefill_custom_voice (src/generate_new.rs:60-188) and build_trailing_text
// (src/generate_new.rs:314-326) on the device.
// ---------------------------------------------------------------------------
namespace {

// Special tokens, src/generate_new.rs:24-36.
constexpr uint32_t kImStart = 151644, kAssistant = 77091, kNewline = 198;
constexpr uint32_t kTtsPad = 151671, kTtsBos = 151672, kTtsEos = 151673;
constexpr uint32_t kCodecThink = 2154, kCodecThinkBos = 2156, kCodecThinkEos = 2157, kCodecPad = 2148,
                   kCodecBos = 2149;
constexpr int kPromptMaxRows = 10;

qtts_status text_reserve(qtts_talker *t, int n) {
    qtts_ctx *c = t->ctx;
    if (!t->has_text) return fail(c, QTTS_ESTATE, "no text weights: call qtts_talker_text_upload first");
    if (n <= t->tx_cap) return QTTS_OK;
    for (void *p : {(void *)t->tx_raw, (void *)t->tx_h, (void *)t->tx_rows, (void *)t->tx_tok})
        if (p) (void)hipFree(p);
    t->tx_raw = t->tx_h = t->tx_rows = nullptr;
    t->tx_tok = nullptr;
    t->tx_cap = 0;
    HIP_TRY(c, hipMalloc(&t->tx_raw, sizeof(float) * n * t->text_hidden));
    HIP_TRY(c, hipMalloc(&t->tx_h, sizeof(float) * n * t->fc1.N));
    HIP_TRY(c, hipMalloc(&t->tx_rows, sizeof(float) * n * t->st.hidden));
    HIP_TRY(c, hipMalloc(&t->tx_tok, sizeof(uint32_t) * n));
    t->tx_cap = n;
    return QTTS_OK;
}

// One layer of the text projection over n rows: y = gemv(x, w) + bias, the
// GEMV with rows of up to kMaxM per launch.
qtts_status text_layer(qtts_talker *t, const DevQ4 &w, const float *x, int n, const float *bias, float *y) {
    for (int r0 = 0; r0 < n; r0 += kMaxM) {
        const int M = n - r0 < kMaxM ? n - r0 : kMaxM;
        GemvParams p = gemv_base(t->ctx, w, M);
        p.prologue = PRO_PLAIN;
        p.x = x + (size_t)r0 * w.K;
        p.ldx = w.K;
        p.epilogue = EPI_STORE;
        p.y = y + (size_t)r0 * w.N;
        p.ldy = w.N;
        p.bias = bias;
        QTTS_TRY(run_gemv(t->ctx, p));
    }
    return QTTS_OK;
}

// embed_text_token of the n host tokens, rows [n][hidden] to `out` (device).
qtts_status text_project(qtts_talker *t, const uint32_t *tokens, int n, float *out) {
    qtts_ctx *c = t->ctx;
    if (!t->has_text) return fail(c, QTTS_ESTATE, "no text weights: call qtts_talker_text_upload first");
    for (int i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)t->text_emb.K) return fail(c, QTTS_ERANGE, "text token id out of range");
    QTTS_TRY(text_reserve(t, n));
    HIP_TRY(c, hipMemcpyAsync(t->tx_tok, tokens, sizeof(uint32_t) * n, hipMemcpyHostToDevice, c->stream));
    launch_embed_rows(c->stream, t->text_emb, t->tx_tok, 1, n, t->tx_raw, t->text_hidden);
    QTTS_TRY(check_launch(c, "k_embed_rows"));
    QTTS_TRY(text_layer(t, t->fc1, t->tx_raw, n, t->fc1_b, t->tx_h));
    launch_silu(c->stream, t->tx_h, (long long)n * t->fc1.N);
    QTTS_TRY(check_launch(c, "k_silu"));
    return text_layer(t, t->fc2, t->tx_h, n, t->fc2_b, out);
}

// The rows of prefill_custom_voice into t->xp (sized for kPromptMaxRows);
// *L = 9 or 10.
qtts_status build_prompt(qtts_talker *t, const uint32_t *text_tokens, int32_t n_text, uint32_t speaker_id,
                         uint32_t language_id, const float *voice, int *L) {
    qtts_ctx *c = t->ctx;
    const int H = t->st.hidden;
    if (n_text < 0 || (n_text > 0 && !text_tokens)) return fail(c, QTTS_EINVAL, "text tokens");
    // text rows: role prefix, TTS_PAD, TTS_BOS, the first text token
    uint32_t tt[6] = {kImStart, kAssistant, kNewline, kTtsPad, kTtsBos, n_text > 0 ? text_tokens[0] : 0u};
    const int nt = n_text > 0 ? 6 : 5;
    // codec rows
    uint32_t ct[7];
    int nc = 0;
    if (voice) {
        const uint32_t v[6] = {kCodecThink, kCodecThinkBos, language_id, kCodecThinkEos, kCodecPad, kCodecBos};
        for (uint32_t x : v) ct[nc++] = x;
    } else {
        const uint32_t v[7] = {kCodecThink, kCodecThinkBos, language_id, kCodecThinkEos, speaker_id, kCodecPad, kCodecBos};
        for (uint32_t x : v) ct[nc++] = x;
    }
    if (n_text == 0) nc--;  // no BOS + first text row
    for (int i = 0; i < nc; i++)
        if (ct[i] >= (uint32_t)t->emb.K) return fail(c, QTTS_ERANGE, "codec token id out of range");
    QTTS_TRY(text_reserve(t, 8));
    float *T = t->tx_rows;  // [TTS role x3, TTS_PAD, TTS_BOS, text[0]]
    QTTS_TRY(text_project(t, tt, nt, T));
    // codec rows (the token buffer is reused in stream order)
    float *codec = t->pr_codec;
    HIP_TRY(c, hipMemcpyAsync(t->tx_tok, ct, sizeof(uint32_t) * nc, hipMemcpyHostToDevice, c->stream));
    launch_embed_rows(c->stream, t->emb, t->tx_tok, 1, nc, codec, H);
    QTTS_TRY(check_launch(c, "k_embed_rows"));
    const float *voice_row = nullptr;
    if (voice) {
        float *vr = codec + (size_t)7 * H;
        HIP_TRY(c, hipMemcpyAsync(vr, voice, sizeof(float) * H, hipMemcpyHostToDevice, c->stream));
        voice_row = vr;
    }
    PromptRowsParams P{};
    int r = 0;
    for (int i = 0; i < 3; i++) P.a[r++] = T + (size_t)i * H;  // role prefix
    const float *pad = T + (size_t)3 * H, *bos = T + (size_t)4 * H;
    if (voice) {
        for (int i = 0; i < 4; i++, r++) {
            P.a[r] = codec + (size_t)i * H;
            P.b[r] = pad;
        }
        P.a[r++] = voice_row;
        P.a[r] = codec + (size_t)4 * H;  // CODEC_PAD
        P.b[r++] = bos;
        if (n_text > 0) {
            P.a[r] = codec + (size_t)5 * H;  // CODEC_BOS
            P.b[r++] = T + (size_t)5 * H;
        }
    } else {
        for (int i = 0; i < 6; i++, r++) {
            P.a[r] = codec + (size_t)i * H;
            P.b[r] = i < 5 ? pad : bos;
        }
        if (n_text > 0) {
            P.a[r] = codec + (size_t)6 * H;  // CODEC_BOS
            P.b[r++] = T + (size_t)5 * H;
        }
    }
    P.L = r;
    P.H = H;
    P.out = t->xp;
    launch_prompt_rows(c->stream, P);
    QTTS_TRY(check_launch(c, "k_prompt_rows"));
    *L = r;
    return QTTS_OK;
}

}  // namespace

qtts_status qtts_talker_text_upload(qtts_talker *t, const qtts_text_view *v) {
    if (!t || !v) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    if (t->has_text) return fail(c, QTTS_ESTATE, "text weights already uploaded");
    const int th = v->text_hidden_size, H = t->st.hidden;
    if (th <= 0) return fail(c, QTTS_ESHAPE, "text_hidden_size must be positive");
    QTTS_TRY(check_view(c, &v->text_embedding, v->text_embedding.k, th, "text_embedding"));
    QTTS_TRY(check_view(c, &v->text_proj_fc1, th, v->text_proj_fc1.n, "text_proj_fc1"));
    QTTS_TRY(check_view(c, &v->text_proj_fc2, v->text_proj_fc1.n, H, "text_proj_fc2"));
    if (v->text_embedding.k <= (int)kTtsEos) return fail(c, QTTS_ESHAPE, "text vocab below the TTS special tokens");
    QTTS_TRY(alloc_q4(c, t->own, v->text_embedding.k, th, &t->text_emb));
    QTTS_TRY(upload_part(c, &v->text_embedding, t->text_emb, 0));
    QTTS_TRY(alloc_q4(c, t->own, th, v->text_proj_fc1.n, &t->fc1));
    QTTS_TRY(upload_part(c, &v->text_proj_fc1, t->fc1, 0));
    QTTS_TRY(alloc_q4(c, t->own, v->text_proj_fc1.n, H, &t->fc2));
    QTTS_TRY(upload_part(c, &v->text_proj_fc2, t->fc2, 0));
    QTTS_TRY(upload_array(c, t->own, v->text_proj_fc1_bias, (size_t)v->text_proj_fc1.n, &t->fc1_b, "text_proj_fc1_bias"));
    QTTS_TRY(upload_array(c, t->own, v->text_proj_fc2_bias, (size_t)H, &t->fc2_b, "text_proj_fc2_bias"));
    QTTS_TRY(t->own.alloc(c, &t->pr_codec, (size_t)8 * H));
    t->text_hidden = th;
    t->has_text = 1;
    return QTTS_OK;
}

qtts_status qtts_embed_text_token(qtts_talker *t, uint32_t token_id, float *out) {
    if (!t || !out) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    QTTS_TRY(text_reserve(t, 1));
    QTTS_TRY(text_project(t, &token_id, 1, t->tx_rows));
    HIP_TRY(c, hipMemcpyAsync(out, t->tx_rows, sizeof(float) * t->st.hidden, hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

qtts_status qtts_build_custom_voice_prompt(qtts_talker *t, const uint32_t *text_tokens, int32_t n_text,
                                           uint32_t speaker_id, uint32_t language_id, const float *voice_embedding,
                                           float *rows, int32_t *seq_len) {
    if (!t || !rows || !seq_len) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    *seq_len = 0;
    QTTS_TRY(prefill_buffers(t, kPromptMaxRows));
    int L = 0;
    QTTS_TRY(build_prompt(t, text_tokens, n_text, speaker_id, language_id, voice_embedding, &L));
    HIP_TRY(c, hipMemcpyAsync(rows, t->xp, sizeof(float) * L * t->st.hidden, hipMemcpyDeviceToHost, c->stream));
    QTTS_TRY(sync(c));
    *seq_len = L;
    return QTTS_OK;
}

qtts_status qtts_prefill_custom_voice(qtts_talker *t, const uint32_t *text_tokens, int32_t n_text, uint32_t speaker_id,
                                      uint32_t language_id, const float *voice_embedding, qtts_kv *kv,
                                      float *last_hidden, float *logits, int32_t *position) {
    if (!t || !kv || !last_hidden || !logits || !position) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    *position = 0;
    const int L = (n_text > 0 ? 1 : 0) + 9;
    QTTS_TRY(prefill_prepare(t, L, kv));
    int built = 0;
    QTTS_TRY(build_prompt(t, text_tokens, n_text, speaker_id, language_id, voice_embedding, &built));
    qtts_status s = prefill_from_xp(t, built, kv);
    if (s != QTTS_OK) {
        kv->len = 0;
        return s;
    }
    const int H = t->st.hidden;
    HIP_TRY(c, hipMemcpyAsync(last_hidden, t->out, sizeof(float) * H, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipMemcpyAsync(logits, t->out + H, sizeof(float) * t->vocab, hipMemcpyDeviceToHost, c->stream));
    QTTS_TRY(sync(c));
    *position = built;  // src/generate_new.rs:216
    return QTTS_OK;
}

qtts_status qtts_prefill_talker(qtts_talker *t, const uint32_t *tokens, const int32_t *is_text, int32_t seq_len,
                                qtts_kv *kv, float *last_hidden) {
    if (!t || !last_hidden || (seq_len > 0 && (!tokens || !is_text))) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    if (seq_len < 1) return fail(c, QTTS_EINVAL, "seq_len < 1");
    // every id checked before any work, so a bad one leaves the cache empty
    std::vector<uint32_t> text_ids, ids((size_t)2 * seq_len);
    int32_t *slot = reinterpret_cast<int32_t *>(ids.data() + seq_len);
    for (int i = 0; i < seq_len; i++) {
        ids[i] = tokens[i];
        if (is_text[i]) {
            if (!t->has_text) return fail(c, QTTS_ESTATE, "text token without text weights: call qtts_talker_text_upload");
            if (tokens[i] >= (uint32_t)t->text_emb.K) return fail(c, QTTS_ERANGE, "text token id out of range");
            slot[i] = (int32_t)text_ids.size();
            text_ids.push_back(tokens[i]);
        } else {
            if (tokens[i] >= (uint32_t)t->emb.K) return fail(c, QTTS_ERANGE, "codec token id out of range");
            slot[i] = -1;
        }
    }
    QTTS_TRY(prefill_prepare(t, seq_len, kv));
    if (seq_len > t->pf_cap) {
        if (t->pf_tok) (void)hipFree(t->pf_tok);
        t->pf_tok = nullptr;
        t->pf_cap = 0;
        HIP_TRY(c, hipMalloc(&t->pf_tok, sizeof(uint32_t) * 2 * seq_len));
        t->pf_cap = seq_len;
    }
    // the text rows in one batch through the projection (embed_text_token,
    // src/talker.rs:105-116), then every row into t->xp in sequence order
    const int nt = (int)text_ids.size();
    if (nt > 0) {
        QTTS_TRY(text_reserve(t, nt));
        QTTS_TRY(text_project(t, text_ids.data(), nt, t->tx_rows));
    }
    HIP_TRY(c, hipMemcpyAsync(t->pf_tok, ids.data(), sizeof(uint32_t) * 2 * seq_len, hipMemcpyHostToDevice, c->stream));
    launch_token_rows(c->stream, t->emb, t->pf_tok, reinterpret_cast<const int *>(t->pf_tok + seq_len), t->tx_rows,
                      seq_len, t->xp, t->st.hidden);
    qtts_status s = check_launch(c, "k_token_rows");
    if (s == QTTS_OK) s = prefill_from_xp(t, seq_len, kv);
    if (s != QTTS_OK) {
        (void)hipStreamSynchronize(c->stream);  // the ids copy reads `ids`
        kv->len = 0;
        return s;
    }
    HIP_TRY(c, hipMemcpyAsync(last_hidden, t->out, sizeof(float) * t->st.hidden, hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

qtts_status qtts_build_trailing_text(qtts_talker *t, const uint32_t *text_tokens, int32_t n_text, float *rows,
                                     int32_t *n_rows) {
    if (!t || !rows || !n_rows || n_text < 0 || (n_text > 0 && !text_tokens)) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    *n_rows = 0;
    std::vector<uint32_t> tok;
    for (int i = 1; i < n_text; i++) tok.push_back(text_tokens[i]);
    tok.push_back(kTtsEos);
    const int n = (int)tok.size();
    QTTS_TRY(text_reserve(t, n));
    QTTS_TRY(text_project(t, tok.data(), n, t->tx_rows));
    HIP_TRY(c, hipMemcpyAsync(rows, t->tx_rows, sizeof(float) * n * t->st.hidden, hipMemcpyDeviceToHost, c->stream));
    QTTS_TRY(sync(c));
    *n_rows = n;
    return QTTS_OK;
}

static qtts_status generate_codes_dev(qtts_talker *t, qtts_predictor *p, qtts_kv *talker_kv, qtts_kv *predictor_kv,
                                      const float *last_hidden, const float *logits, int32_t position,
                                      const float *trailing_text, int32_t trailing_len, const float *tts_pad_embed,
                                      const qtts_loop_params *params, uint64_t seed, uint32_t *codes,
                                      int32_t *n_frames);

// generate_speech up to the codes (src/generate_new.rs:205-300).  With codes
// NULL the codes stay in t->codes ([16][params->max_codes], frame-minor) only.
static qtts_status speech_codes(qtts_talker *t, qtts_predictor *p, const uint32_t *text_tokens, int32_t n_text,
                                uint32_t speaker_id, uint32_t language_id, const float *voice_embedding,
                                qtts_kv *talker_kv, qtts_kv *predictor_kv, const qtts_loop_params *params,
                                uint64_t seed, uint32_t *codes, int32_t *n_frames) {
    if (!t || !talker_kv || !params || !n_frames) return QTTS_EINVAL;
    *n_frames = 0;
    const int H = t->st.hidden;
    std::vector<float> last_hidden(H), logits(t->vocab), pad(H);
    std::vector<float> trailing((size_t)(n_text > 1 ? n_text : 1) * H);
    int32_t position = 0, rows = 0;
    QTTS_TRY(qtts_prefill_custom_voice(t, text_tokens, n_text, speaker_id, language_id, voice_embedding, talker_kv,
                                       last_hidden.data(), logits.data(), &position));
    QTTS_TRY(qtts_build_trailing_text(t, text_tokens, n_text, trailing.data(), &rows));
    QTTS_TRY(qtts_embed_text_token(t, kTtsPad, pad.data()));
    return generate_codes_dev(t, p, talker_kv, predictor_kv, last_hidden.data(), logits.data(), position,
                              trailing.data(), rows, pad.data(), params, seed, codes, n_frames);
}

qtts_status qtts_generate_speech_codes(qtts_talker *t, qtts_predictor *p, const uint32_t *text_tokens, int32_t n_text,
                                       uint32_t speaker_id, uint32_t language_id, const float *voice_embedding,
                                       qtts_kv *talker_kv, qtts_kv *predictor_kv, const qtts_loop_params *params,
                                       uint64_t seed, uint32_t *codes, int32_t *n_frames) {
    if (!codes) return QTTS_EINVAL;
    return speech_codes(t, p, text_tokens, n_text, speaker_id, language_id, voice_embedding, talker_kv, predictor_kv,
                        params, seed, codes, n_frames);
}

qtts_status qtts_forward_talker_decode(qtts_talker *t, uint32_t token_id, int32_t is_text, qtts_kv *kv,
                                       int32_t position, float *hidden) {
    if (!t || !hidden) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    QTTS_TRY(talker_step_check(t, kv, position));
    if (is_text) {
        QTTS_TRY(text_project(t, &token_id, 1, t->x));
    } else {
        if (token_id >= (uint32_t)t->emb.K) return fail(c, QTTS_ERANGE, "token id out of range");
        HIP_TRY(c, hipMemcpyAsync(c->d_small, &token_id, 4, hipMemcpyHostToDevice, c->stream));
        launch_embed_row(c->stream, t->emb, c->d_small, t->x, nullptr);
        QTTS_TRY(check_launch(c, "k_embed_row"));
    }
    return talker_step_x(t, kv, position, hidden, t->st.hidden);
}

// ---------------------------------------------------------------------------
qtts_status qtts_predictor_upload(qtts_ctx *c, const qtts_predictor_view *v, qtts_predictor **out) {
    if (!c || !v || !out) return QTTS_EINVAL;
    *out = nullptr;
    if (v->num_groups <= 0 || v->num_groups > kMaxGroups) return fail(c, QTTS_ESHAPE, "num_groups must be 1..15");
    if (!v->codec_embeddings || !v->lm_heads) return fail(c, QTTS_EINVAL, "null embeddings or heads");
    qtts_predictor *p = new qtts_predictor();
    p->ctx = ctx_retain(c);
    auto bail = [&](qtts_status s) {
        delete p;
        return s;
    };
    const int hidden = v->hidden_size;
    qtts_status s =
        upload_stack(c, p->own, v->num_layers, v->layers, hidden, v->num_heads, v->num_kv_heads, v->head_dim, &p->st);
    if (s != QTTS_OK) return bail(s);
    p->groups = v->num_groups;
    p->embed_dim = v->codec_embeddings[0].n;
    p->vocab = v->lm_heads[0].n;
    p->identity_proj = v->input_proj.k == 0;
    p->talker_hidden = p->identity_proj ? hidden : v->input_proj.k;
    if (p->embed_dim != p->talker_hidden)
        return bail(fail(c, QTTS_ESHAPE, "codec embedding width must equal the projection input"));
    if (!p->identity_proj) {
        if ((s = check_view(c, &v->input_proj, p->talker_hidden, hidden, "input_proj")) != QTTS_OK) return bail(s);
        if ((s = alloc_q4(c, p->own, p->talker_hidden, hidden, &p->in_proj)) != QTTS_OK) return bail(s);
        if ((s = upload_part(c, &v->input_proj, p->in_proj, 0)) != QTTS_OK) return bail(s);
        if (v->input_proj_bias &&
            (s = upload_array(c, p->own, v->input_proj_bias, (size_t)hidden, &p->bias, "input_proj_bias")) != QTTS_OK)
            return bail(s);
    }
    for (int g = 0; g < p->groups; g++) {
        const qtts_q4_view &e = v->codec_embeddings[g];
        if ((s = check_view(c, &e, e.k, p->embed_dim, "codec_embeddings")) != QTTS_OK) return bail(s);
        if ((s = alloc_q4(c, p->own, e.k, p->embed_dim, &p->emb[g])) != QTTS_OK) return bail(s);
        if ((s = upload_part(c, &e, p->emb[g], 0)) != QTTS_OK) return bail(s);
        const qtts_q4_view &h = v->lm_heads[g];
        if ((s = check_view(c, &h, hidden, p->vocab, "lm_heads")) != QTTS_OK) return bail(s);
        if ((s = alloc_q4(c, p->own, hidden, p->vocab, &p->heads[g])) != QTTS_OK) return bail(s);
        if ((s = upload_part(c, &h, p->heads[g], 0)) != QTTS_OK) return bail(s);
    }
    if ((s = upload_array(c, p->own, v->final_norm_gamma, (size_t)hidden, &p->st.final_g, "final_norm_gamma")) !=
        QTTS_OK)
        return bail(s);
    // The whole table, as src/loader.rs:859-874 builds it (65536 rows for
    // the 1.7B model, 32 MiB): generate_acoustic_codes only reaches
    // positions 0..num_groups, but predict_codes keeps appending to its
    // cache.  Positions past the table skip the rotation, as
    // src/code_predictor.rs:107 does.
    const int rows = v->max_position;
    p->max_pos = v->max_position;
    if (rows < 1) return bail(fail(c, QTTS_EINVAL, "max_position must be positive"));
    if ((s = upload_rope(c, p->own, v->head_dim, rows, v->rope_theta, v->rope_cos, v->rope_sin, &p->st)) != QTTS_OK) return bail(s);
    p->st.rope_skip_oob = 1;
    const int qd = p->st.nq * p->st.hd;
    if ((s = p->own.alloc(c, &p->in2, 2 * (size_t)p->talker_hidden)) != QTTS_OK) return bail(s);
    if ((s = p->own.alloc(c, &p->x2, 2 * (size_t)hidden)) != QTTS_OK) return bail(s);
    if ((s = p->own.alloc(c, &p->q2, 2 * (size_t)qd)) != QTTS_OK) return bail(s);
    if ((s = p->own.alloc(c, &p->a2, 2 * (size_t)qd)) != QTTS_OK) return bail(s);
    if ((s = p->own.alloc(c, &p->h2, 2 * (size_t)p->st.inter)) != QTTS_OK) return bail(s);
    if ((s = p->own.alloc(c, &p->logits, (size_t)p->vocab)) != QTTS_OK) return bail(s);
    if ((s = p->own.alloc(c, &p->codes, 16)) != QTTS_OK) return bail(s);
    if ((s = p->own.alloc(c, &p->status, 4)) != QTTS_OK) return bail(s);
    *out = p;
    return QTTS_OK;
}

void qtts_predictor_free(qtts_predictor *p) {
    if (!p) return;
    qtts_ctx *c = p->ctx;
    if (c) (void)hipStreamSynchronize(c->stream);
    delete p;
    if (c) ctx_release(c);
}

namespace {

// generate_acoustic_codes (src/code_predictor.rs:218-273) on device buffers:
// p->in2 = [talker_hidden; semantic_embed]; the 15 codes go to codes_out.
qtts_status enqueue_predictor(qtts_predictor *p, qtts_kv *kv, uint32_t *codes_out, int *status, const int *d_done) {
    qtts_ctx *c = p->ctx;
    const Stack &st = p->st;
    const int hidden = st.hidden;
    const int nsplit = attn_nsplit(kv->cap, 1);
    // 1. project both prefill rows
    if (p->identity_proj) {
        HIP_TRY(c, hipMemcpyAsync(p->x2, p->in2, sizeof(float) * 2 * hidden, hipMemcpyDeviceToDevice, c->stream));
    } else {
        GemvParams g = gemv_base(c, p->in_proj, 2);
        g.prologue = PRO_PLAIN;
        g.x = p->in2;
        g.ldx = p->talker_hidden;
        g.epilogue = EPI_STORE;
        g.y = p->x2;
        g.ldy = hidden;
        g.bias = p->bias;
        g.d_done = d_done;
        QTTS_TRY(run_gemv(c, g));
    }
    // 2. two-token prefill at positions 0, 1
    QTTS_TRY(enqueue_layers(c, st, kv, p->x2, p->q2, p->a2, p->h2, 2, nullptr, 0, nullptr, 0, nsplit, d_done));
    auto head = [&](int gi, int src_row) -> qtts_status {
        GemvParams g = gemv_base(c, p->heads[gi], 1);
        g.prologue = PRO_RMSNORM;
        g.x = p->x2;
        g.ldx = hidden;
        g.norm_src_row0 = src_row;
        g.gamma = st.final_g;
        g.epilogue = EPI_STORE;
        g.y = p->logits;
        g.ldy = p->vocab;
        g.fin = FIN_ARGMAX;
        g.argmax_out = codes_out + gi;
        g.status = status;
        g.d_done = d_done;
        return run_gemv(c, g);
    };
    QTTS_TRY(head(0, 1));
    // 3. fourteen single-token decodes at cache offsets 2..15
    for (int gi = 1; gi < p->groups; gi++) {
        if (p->identity_proj) {
            launch_embed_row(c->stream, p->emb[gi - 1], codes_out + gi - 1, p->x2, d_done);
            QTTS_TRY(check_launch(c, "k_embed_row"));
        } else {
            GemvParams g = gemv_base(c, p->in_proj, 1);
            g.prologue = PRO_EMBED;
            g.emb = p->emb[gi - 1];
            g.emb_token = codes_out + gi - 1;
            g.epilogue = EPI_STORE;
            g.y = p->x2;
            g.ldy = hidden;
            g.bias = p->bias;
            g.d_done = d_done;
            QTTS_TRY(run_gemv(c, g));
        }
        QTTS_TRY(enqueue_layers(c, st, kv, p->x2, p->q2, p->a2, p->h2, 1, nullptr, gi + 1, nullptr, gi + 1, nsplit,
                                d_done));
        QTTS_TRY(head(gi, 0));
    }
    return QTTS_OK;
}

}  // namespace

qtts_status qtts_generate_acoustic_codes(qtts_predictor *p, const float *talker_hidden, const float *semantic_embed,
                                         qtts_kv *kv, uint32_t *codes) {
    if (!p || !talker_hidden || !semantic_embed || !codes) return QTTS_EINVAL;
    qtts_ctx *c = p->ctx;
    QTTS_TRY(check_kv(c, p->st, kv));
    if (kv->cap < p->groups + 1) return fail(c, QTTS_ERANGE, "predictor cache needs num_groups+1 positions");
    kv->len = 0;  // src/code_predictor.rs:227-231
    const int th = p->talker_hidden;
    HIP_TRY(c, hipMemcpyAsync(p->in2, talker_hidden, sizeof(float) * th, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipMemcpyAsync(p->in2 + th, semantic_embed, sizeof(float) * th, hipMemcpyHostToDevice, c->stream));
    if (engine_enabled() && !p->identity_proj) {
        QTTS_TRY(eng_init(c));
        if (!p->prog || p->prog_kv != kv->serial) {
            p->prog.reset(new EngProgram());
            QTTS_TRY(eng_build(c, *p->prog, [&](EngProgram &P) {
                TvRef codes[kMaxGroups];
                return build_predictor_passes(P, p, kv, in_plain(p->in2), in_plain(p->in2 + th), codes);
            }));
            p->prog_kv = kv->serial;
        }
        if (!p->prog->unsupported) {
            QTTS_TRY(eng_reset(c, 0, 0, 0));
            QTTS_TRY(eng_launch(c, *p->prog, 0, p->codes, 1));
            uint32_t all[16];
            HIP_TRY(c, hipMemcpyAsync(all, p->codes, sizeof(all), hipMemcpyDeviceToHost, c->stream));
            QTTS_TRY(sync(c));
            QTTS_TRY(eng_status_check(c, "generate_acoustic_codes"));
            for (int g = 0; g < p->groups; g++) codes[g] = all[1 + g];
            kv->len = p->groups + 1;
            return QTTS_OK;
        }
    }
    HIP_TRY(c, hipMemsetAsync(p->status, 0, sizeof(int), c->stream));
    QTTS_TRY(enqueue_predictor(p, kv, p->codes, p->status, nullptr));
    int status = 0;
    HIP_TRY(c, hipMemcpyAsync(codes, p->codes, sizeof(uint32_t) * p->groups, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(c, hipMemcpyAsync(&status, p->status, sizeof(int), hipMemcpyDeviceToHost, c->stream));
    QTTS_TRY(sync(c));
    kv->len = p->groups + 1;
    if (status != 0) return fail(c, (qtts_status)status, "NaN logits in the predictor (src/code_predictor.rs:331)");
    return QTTS_OK;
}

qtts_status qtts_predict_codes(qtts_predictor *p, const float *talker_hidden, qtts_kv *kv, float *logits) {
    if (!p || !talker_hidden || !logits) return QTTS_EINVAL;
    qtts_ctx *c = p->ctx;
    QTTS_TRY(check_kv(c, p->st, kv));
    const int offset = kv->len, H = p->st.hidden;
    if (offset + 1 > kv->cap) return fail(c, QTTS_ERANGE, "predictor cache full");
    const size_t nlog = (size_t)p->groups * p->vocab;
    QTTS_TRY(ensure_staging(c, 0, nlog));
    HIP_TRY(c, hipMemcpyAsync(p->in2, talker_hidden, sizeof(float) * p->talker_hidden, hipMemcpyHostToDevice,
                              c->stream));
    // project_input (src/code_predictor.rs:51-61)
    if (p->identity_proj) {
        HIP_TRY(c, hipMemcpyAsync(p->x2, p->in2, sizeof(float) * H, hipMemcpyDeviceToDevice, c->stream));
    } else {
        GemvParams g = gemv_base(c, p->in_proj, 1);
        g.prologue = PRO_PLAIN;
        g.x = p->in2;
        g.ldx = p->talker_hidden;
        g.epilogue = EPI_STORE;
        g.y = p->x2;
        g.ldy = H;
        g.bias = p->bias;
        QTTS_TRY(run_gemv(c, g));
    }
    // one decode step at the cache offset (RoPE at the offset,
    // src/code_predictor.rs:147-156), then every head on the final-normed row
    QTTS_TRY(enqueue_layers(c, p->st, kv, p->x2, p->q2, p->a2, p->h2, 1, nullptr, offset, nullptr, offset,
                            attn_nsplit(kv->cap, 1), nullptr));
    for (int g = 0; g < p->groups; g++) {
        GemvParams q = gemv_base(c, p->heads[g], 1);
        q.prologue = PRO_RMSNORM;
        q.x = p->x2;
        q.ldx = H;
        q.gamma = p->st.final_g;
        q.epilogue = EPI_STORE;
        q.y = c->d_out + (size_t)g * p->vocab;
        q.ldy = p->vocab;
        QTTS_TRY(run_gemv(c, q));
    }
    HIP_TRY(c, hipMemcpyAsync(logits, c->d_out, sizeof(float) * nlog, hipMemcpyDeviceToHost, c->stream));
    QTTS_TRY(sync(c));
    kv->len = offset + 1;
    return QTTS_OK;
}

qtts_status qtts_get_acoustic_embeddings_sum(qtts_predictor *p, const uint32_t *codes, float *out) {
    if (!p || !codes || !out) return QTTS_EINVAL;
    qtts_ctx *c = p->ctx;
    for (int g = 0; g < p->groups; g++)
        if (codes[g] >= (uint32_t)p->emb[g].K) return fail(c, QTTS_ERANGE, "code out of range");
    uint32_t cur[16] = {0};
    for (int g = 0; g < p->groups; g++) cur[1 + g] = codes[g];
    QTTS_TRY(ensure_staging(c, 0, (size_t)p->embed_dim));
    HIP_TRY(c, hipMemcpyAsync(p->codes, cur, sizeof(cur), hipMemcpyHostToDevice, c->stream));
    EmbSumParams e{};
    e.mode = 1;
    for (int g = 0; g < p->groups; g++) e.group_emb[g] = p->emb[g];
    e.num_groups = p->groups;
    e.cur = p->codes;
    e.out = c->d_out;
    e.hidden = p->embed_dim;
    launch_embed_sum(c->stream, e);
    QTTS_TRY(check_launch(c, "k_embed_sum"));
    HIP_TRY(c, hipMemcpyAsync(out, c->d_out, sizeof(float) * p->embed_dim, hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

// ---------------------------------------------------------------------------
qtts_status qtts_sample_token(qtts_ctx *c, const float *logits, int32_t vocab, const qtts_sampler *params,
                              const uint32_t *prev_tokens, int32_t n_prev, uint64_t *rng, uint32_t *token) {
    if (!c || !logits || !params || !rng || !token || (n_prev > 0 && !prev_tokens)) return QTTS_EINVAL;
    if (vocab <= 0 || vocab > 32768) return fail(c, QTTS_ESHAPE, "vocab must be 1..32768");
    if (n_prev < 0 || n_prev > 32) return fail(c, QTTS_EINVAL, "n_prev must be 0..32");
    QTTS_TRY(ensure_staging(c, (size_t)vocab, 0));
    // d_small layout: [0] token, [1] status, [2..3] rng, [4..35] prev tokens
    uint32_t small[36] = {0};
    std::memcpy(&small[2], rng, 8);
    if (n_prev > 0) std::memcpy(&small[4], prev_tokens, sizeof(uint32_t) * n_prev);
    HIP_TRY(c, hipMemcpyAsync(c->d_in, logits, sizeof(float) * vocab, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipMemcpyAsync(c->d_small, small, sizeof(small), hipMemcpyHostToDevice, c->stream));
    SampleParams s{};
    s.logits = c->d_in;
    s.vocab = vocab;
    s.temperature = params->temperature;
    s.top_k = params->top_k;
    s.penalty = params->repetition_penalty;
    s.greedy = params->greedy;
    s.prev = c->d_small + 4;
    s.n_prev = n_prev;
    s.rng = reinterpret_cast<uint64_t *>(c->d_small + 2);
    s.token_out = c->d_small;
    s.status = reinterpret_cast<int *>(c->d_small + 1);
    launch_sample(c->stream, s);
    QTTS_TRY(check_launch(c, "k_sample"));
    HIP_TRY(c, hipMemcpyAsync(small, c->d_small, 16, hipMemcpyDeviceToHost, c->stream));
    QTTS_TRY(sync(c));
    *token = small[0];
    std::memcpy(rng, &small[2], 8);
    if (small[1] != 0) return fail(c, (qtts_status)small[1], "NaN in the sampler (src/generate_new.rs:365)");
    return QTTS_OK;
}

qtts_status qtts_sample_top_k(qtts_ctx *c, const float *logits, int32_t vocab, float temperature, int32_t top_k,
                              uint64_t *rng, uint32_t *token) {
    if (!c || !logits || !rng || !token) return QTTS_EINVAL;
    if (vocab <= 0 || vocab > kTopKMaxVocab) return fail(c, QTTS_ESHAPE, "sample_top_k: vocab must be 1..4096");
    if (temperature > 0.0f && top_k < 1) return fail(c, QTTS_EINVAL, "sample_top_k: top_k < 1 (the reference panics)");
    QTTS_TRY(ensure_staging(c, (size_t)vocab, 0));
    // d_small: [0] token, [1] status, [2..3] rng
    uint32_t small[4] = {0, 0, 0, 0};
    std::memcpy(&small[2], rng, 8);
    HIP_TRY(c, hipMemcpyAsync(c->d_in, logits, sizeof(float) * vocab, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipMemcpyAsync(c->d_small, small, sizeof(small), hipMemcpyHostToDevice, c->stream));
    TopKParams P{};
    P.logits = c->d_in;
    P.vocab = vocab;
    P.temperature = temperature;
    P.top_k = top_k;
    P.rng = reinterpret_cast<uint64_t *>(c->d_small + 2);
    P.token_out = c->d_small;
    P.status = reinterpret_cast<int *>(c->d_small + 1);
    launch_sample_top_k(c->stream, P);
    QTTS_TRY(check_launch(c, "k_sample_top_k"));
    HIP_TRY(c, hipMemcpyAsync(small, c->d_small, sizeof(small), hipMemcpyDeviceToHost, c->stream));
    QTTS_TRY(sync(c));
    if (small[1] != 0) return fail(c, (qtts_status)small[1], "sample_top_k: NaN logits (the reference panics)");
    *token = small[0];
    std::memcpy(rng, &small[2], 8);
    return QTTS_OK;
}

// ---------------------------------------------------------------------------
// Frame loop
// ---------------------------------------------------------------------------
namespace {

struct LoopCfg {
    qtts_talker *t;
    qtts_predictor *p;
    qtts_kv *tkv, *pkv;
    const qtts_loop_params *params;
    int trailing_len;
};

// One frame of src/generate_new.rs:242-300 on the device.
qtts_status enqueue_frame(const LoopCfg &L) {
    qtts_talker *t = L.t;
    qtts_ctx *c = t->ctx;
    LoopState *S = t->state;
    const int hidden = t->st.hidden;
    const bool talker_only = L.params->talker_only || !L.p;
    SampleParams s{};
    s.logits = t->out + hidden;
    s.vocab = t->vocab;
    s.temperature = L.params->sampler.temperature;
    s.top_k = L.params->sampler.top_k;
    s.penalty = L.params->sampler.repetition_penalty;
    s.greedy = L.params->sampler.greedy;
    s.prev = S->prev;
    s.n_prev = 16;
    s.rng = &S->rng;
    s.token_out = &S->cur[0];
    s.status = &S->status;
    s.done = &S->done;
    s.stop_on_eos = L.params->stop_on_eos;
    s.eos = L.params->codec_eos_id;
    s.codes = t->codes;
    s.frame = &S->frame;
    s.max_codes = L.params->max_codes;
    s.prev_out = &S->prev[0];
    launch_sample(c->stream, s);
    QTTS_TRY(check_launch(c, "k_sample"));
    EmbSumParams e{};
    e.mode = 0;
    e.codec_emb = t->emb;
    e.cur = S->cur;
    e.trailing = t->trailing;
    e.trailing_len = L.trailing_len;
    e.pad = t->pad;
    e.frame = &S->frame;
    e.out = t->x;
    e.hidden = hidden;
    e.d_done = &S->done;
    e.codes = t->codes;
    e.max_codes = L.params->max_codes;
    e.prev = S->prev;
    float *hidden_out = t->out;
    if (!talker_only) {
        qtts_predictor *p = L.p;
        launch_embed_row(c->stream, t->emb, &S->cur[0], p->in2 + p->talker_hidden, &S->done);
        QTTS_TRY(check_launch(c, "k_embed_row"));
        QTTS_TRY(enqueue_predictor(p, L.pkv, &S->cur[1], &S->status, &S->done));
        for (int g = 0; g < p->groups; g++) e.group_emb[g] = p->emb[g];
        e.num_groups = p->groups;
        hidden_out = p->in2;  // next frame's predictor input row 0
    }
    launch_embed_sum(c->stream, e);
    QTTS_TRY(check_launch(c, "k_embed_sum"));
    return enqueue_talker_step(t, L.tkv, hidden_out, t->out + hidden, &S->done, 1);
}

}  // namespace

qtts_status qtts_generate_codes(qtts_talker *t, qtts_predictor *p, qtts_kv *talker_kv, qtts_kv *predictor_kv,
                                const float *last_hidden, const float *logits, int32_t position,
                                const float *trailing_text, int32_t trailing_len, const float *tts_pad_embed,
                                const qtts_loop_params *params, uint64_t seed, uint32_t *codes, int32_t *n_frames) {
    if (!codes) return QTTS_EINVAL;
    return generate_codes_dev(t, p, talker_kv, predictor_kv, last_hidden, logits, position, trailing_text,
                              trailing_len, tts_pad_embed, params, seed, codes, n_frames);
}

// The frame loop of qtts_generate_codes; with codes NULL the codes stay in
// t->codes ([16][params->max_codes], frame-minor) and are not copied out.
static qtts_status generate_codes_dev(qtts_talker *t, qtts_predictor *p, qtts_kv *talker_kv, qtts_kv *predictor_kv,
                                      const float *last_hidden, const float *logits, int32_t position,
                                      const float *trailing_text, int32_t trailing_len, const float *tts_pad_embed,
                                      const qtts_loop_params *params, uint64_t seed, uint32_t *codes,
                                      int32_t *n_frames) {
    if (!t || !last_hidden || !logits || !params || !n_frames) return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    *n_frames = 0;
    const bool talker_only = params->talker_only || !p;
    if (!talker_only && (!predictor_kv || !tts_pad_embed || (trailing_len > 0 && !trailing_text)))
        return fail(c, QTTS_EINVAL, "predictor loop needs a predictor cache, tts_pad_embed and trailing text");
    if (trailing_len < 0) return fail(c, QTTS_EINVAL, "trailing_len < 0");
    QTTS_TRY(check_kv(c, t->st, talker_kv));
    if (!talker_only) {
        QTTS_TRY(check_kv(c, p->st, predictor_kv));
        if (predictor_kv->cap < p->groups + 1) return fail(c, QTTS_ERANGE, "predictor cache too small");
        if (p->talker_hidden != t->st.hidden) return fail(c, QTTS_ESHAPE, "predictor input width != talker hidden");
    }
    const int max_codes = params->max_codes;
    if (max_codes <= 0) return QTTS_OK;
    if (position < 0 || position + max_codes > t->max_pos) return fail(c, QTTS_ERANGE, "positions beyond the RoPE table");
    if (talker_kv->len + max_codes > talker_kv->cap) return fail(c, QTTS_ERANGE, "talker cache too small");
    const int hidden = t->st.hidden;
    t->nsplit = attn_nsplit_row(talker_kv->cap);
    // device buffers
    const size_t ncodes = (size_t)16 * max_codes;
    if (ncodes > t->codes_cap) {
        if (t->codes) (void)hipFree(t->codes);
        t->codes = nullptr;
        t->codes_cap = 0;
        HIP_TRY(c, hipMalloc(&t->codes, ncodes * sizeof(uint32_t)));
        t->codes_cap = ncodes;
    }
    HIP_TRY(c, hipMemsetAsync(t->codes, 0, ncodes * sizeof(uint32_t), c->stream));
    const size_t ntrail = (size_t)(trailing_len > 0 ? trailing_len : 1) * hidden;
    if (ntrail > t->trailing_cap) {
        if (t->trailing) (void)hipFree(t->trailing);
        t->trailing = nullptr;
        t->trailing_cap = 0;
        HIP_TRY(c, hipMalloc(&t->trailing, ntrail * sizeof(float)));
        t->trailing_cap = ntrail;
    }
    if (trailing_len > 0)
        HIP_TRY(c, hipMemcpyAsync(t->trailing, trailing_text, sizeof(float) * trailing_len * hidden,
                                  hipMemcpyHostToDevice, c->stream));
    if (tts_pad_embed)
        HIP_TRY(c, hipMemcpyAsync(t->pad, tts_pad_embed, sizeof(float) * hidden, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipMemcpyAsync(t->out + hidden, logits, sizeof(float) * t->vocab, hipMemcpyHostToDevice, c->stream));
    if (!talker_only)
        HIP_TRY(c, hipMemcpyAsync(p->in2, last_hidden, sizeof(float) * hidden, hipMemcpyHostToDevice, c->stream));
    LoopState init{};
    init.pos = position;
    init.kvlen = talker_kv->len;
    init.rng = seed;
    HIP_TRY(c, hipMemcpyAsync(t->state, &init, sizeof(init), hipMemcpyHostToDevice, c->stream));
    QTTS_TRY(sync(c));

    bool eng_ok = false;  // the frame program is built and runs in k_engine
    if (engine_enabled() && eng_talker_fits(talker_kv->cap) && (talker_only || !p->identity_proj) &&
        t->vocab <= 4096) {
        QTTS_TRY(eng_init(c));
        char key[256];
        std::snprintf(key, sizeof(key), "%llu %llu %llu %d %d %g %d %g %d %u %d %d %p %p",
                      (unsigned long long)talker_kv->serial, (unsigned long long)(predictor_kv ? predictor_kv->serial : 0),
                      (unsigned long long)(talker_only ? 0 : p->serial), max_codes, trailing_len,
                      params->sampler.temperature, params->sampler.top_k, params->sampler.repetition_penalty,
                      params->sampler.greedy, params->codec_eos_id, params->stop_on_eos, (int)talker_only,
                      (void *)t->trailing, (void *)t->codes);
        if (!t->frame_prog || t->frame_key != key) {
            t->frame_prog.reset(new EngProgram());
            const int nsplit = eng_talker_nsplit(talker_kv->cap);
            QTTS_TRY(eng_build(c, *t->frame_prog, [&](EngProgram &P) {
                EngOp op{};
                op.kind = EOP_SAMPLE;
                op.ntasks = 1;
                EngSample &sm = op.samp;
                sm.logits = t->out + hidden;
                sm.vocab = t->vocab;
                sm.temperature = params->sampler.temperature;
                sm.top_k = params->sampler.top_k;
                sm.penalty = params->sampler.repetition_penalty;
                sm.greedy = params->sampler.greedy;
                sm.stop_on_eos = params->stop_on_eos;
                sm.eos = params->codec_eos_id;
                sm.num_prev = 16;
                sm.tok = P.tv(1);
                sm.tok_tag = P.tag();
                P.push(op);
                const TvRef tok{sm.tok, sm.tok_tag, 1};
                TvRef x;
                if (!talker_only) {
                    TvRef codes[kMaxGroups];
                    QTTS_TRY(build_predictor_passes(P, p, predictor_kv, in_plain(t->out), in_embed(t->emb, tok), codes));
                    x = add_embsum(P, 0, &t->emb, p->emb, codes, p->groups, tok, t->trailing, trailing_len, t->pad,
                                   hidden);
                } else {
                    x = add_embsum(P, 1, &t->emb, nullptr, nullptr, 0, tok, nullptr, 0, nullptr, hidden);
                }
                return build_talker_layers_and_head(P, t, talker_kv, x, nsplit);
            }));
            t->frame_key = key;
        }
        eng_ok = !t->frame_prog->unsupported;
    }
    if (eng_ok) {
        // t->out holds [last_hidden | logits] for the first frame's sampler
        // and predictor input.
        HIP_TRY(c, hipMemcpyAsync(t->out, last_hidden, sizeof(float) * hidden, hipMemcpyHostToDevice, c->stream));
        QTTS_TRY(eng_reset(c, position, talker_kv->len, seed));
        qtts_status rc = QTTS_OK;
        const int batch = 16;
        int done = 0;
        for (int f0 = 0; f0 < max_codes && rc == QTTS_OK && !done; f0 += batch) {
            const int nb = max_codes - f0 < batch ? max_codes - f0 : batch;
            rc = eng_launch(c, *t->frame_prog, f0 & 1, t->codes, max_codes, nb);
            if (rc != QTTS_OK) break;
            if (params->stop_on_eos && f0 + nb < max_codes) {
                int d = 0;
                hipError_t e = hipMemcpyAsync(&d, c->eng_done, sizeof(int), hipMemcpyDeviceToHost, c->stream);
                if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
                if (e != hipSuccess) rc = fail(c, QTTS_EDEVICE, std::string("loop: ") + hipGetErrorString(e));
                done = d;
            }
        }
        QTTS_TRY(rc);
        QTTS_TRY(sync(c));
        QTTS_TRY(eng_status_check(c, "generate_codes"));
        EngState fin[2];
        HIP_TRY(c, hipMemcpy(fin, c->eng_state, sizeof(fin), hipMemcpyDeviceToHost));
        if (codes) HIP_TRY(c, hipMemcpy(codes, t->codes, ncodes * sizeof(uint32_t), hipMemcpyDeviceToHost));
        const int nf = fin[0].frame > fin[1].frame ? fin[0].frame : fin[1].frame;
        *n_frames = nf;
        talker_kv->len += nf;
        if (!talker_only && nf > 0) predictor_kv->len = p->groups + 1;
        return QTTS_OK;
    }

    LoopCfg L{t, talker_only ? nullptr : p, talker_kv, predictor_kv, params, trailing_len};
    const bool use_graph = std::getenv("QTTS_NO_GRAPH") == nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    if (use_graph) {
        HIP_TRY(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        qtts_status s = enqueue_frame(L);
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamEndCapture(c->stream, &g);
        if (s != QTTS_OK) {
            if (g) (void)hipGraphDestroy(g);
            return s;
        }
        if (e != hipSuccess) return fail(c, QTTS_EDEVICE, std::string("graph capture: ") + hipGetErrorString(e));
        graph = g;
        e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(graph);
            return fail(c, QTTS_EDEVICE, std::string("graph instantiate: ") + hipGetErrorString(e));
        }
    }
    qtts_status rc = QTTS_OK;
    const int batch = 16;
    LoopState fin{};
    for (int f0 = 0; f0 < max_codes && rc == QTTS_OK; f0 += batch) {
        const int nb = max_codes - f0 < batch ? max_codes - f0 : batch;
        for (int i = 0; i < nb && rc == QTTS_OK; i++) {
            if (use_graph) {
                hipError_t e = hipGraphLaunch(exec, c->stream);
                if (e != hipSuccess) rc = fail(c, QTTS_EDEVICE, std::string("graph launch: ") + hipGetErrorString(e));
            } else {
                rc = enqueue_frame(L);
            }
        }
        if (rc != QTTS_OK) break;
        hipError_t e = hipMemcpyAsync(&fin, t->state, sizeof(fin), hipMemcpyDeviceToHost, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) {
            rc = fail(c, QTTS_EDEVICE, std::string("loop: ") + hipGetErrorString(e));
            break;
        }
        if (fin.done) break;
    }
    // No replay may still be in flight when the executable graph goes away.
    if (rc != QTTS_OK) (void)hipStreamSynchronize(c->stream);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    QTTS_TRY(rc);
    QTTS_TRY(sync(c));
    // A failed loop (NaN logits: the reference panics) leaves the caches'
    // lengths and *n_frames as they were, as the frame engine does.
    if (fin.status != 0) return fail(c, (qtts_status)fin.status, "generate_codes: NaN logits (the reference panics)");
    if (codes) HIP_TRY(c, hipMemcpy(codes, t->codes, ncodes * sizeof(uint32_t), hipMemcpyDeviceToHost));
    *n_frames = fin.frame;
    talker_kv->len += fin.frame;
    if (!talker_only && fin.frame > 0) predictor_kv->len = p->groups + 1;
    return QTTS_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Speech decoder: decode_to_audio (src/decoder.rs:394-509) on the device.
// The weights keep the reference's layouts; every projection and convolution
// runs on the matrix cores (k_dec_conv_mfma, csrc/decoder.hip) from a
// binary16 hi + lo operand copy made at upload.
// ---------------------------------------------------------------------------
// A convolution's or linear layer's weights as binary16 hi + lo
// matrix-core operands (DecConvMfmaParams).
struct DecConvMfma {
    _Float16 *wh = nullptr, *wl = nullptr;
    int ew = 0, mtiles = 0, ksteps = 0, cin16 = 0;
};

struct qtts_decoder {
    qtts_ctx *ctx = nullptr;
    Owner own;
    // the Vocos convolutions on the matrix cores: [block][unit][conv1, conv2]
    // and [block][output phase] of each block's transposed convolution
    std::vector<std::vector<std::array<DecConvMfma, 2>>> res_mfma;
    std::vector<std::vector<DecConvMfma>> up_mfma;
    // the other matrix-core layers: codebook projections, pre-conv, the
    // transformer's input / output and per-layer q, k, v, o, gate, up, down,
    // each ConvNeXt stage's transposed convolution (per phase) and pw1, pw2,
    // the Vocos input and output convolutions
    DecConvMfma proj0, proj_rest, pre_conv, tf_in, tf_out, vocos_init, out_conv;
    std::vector<std::array<DecConvMfma, 7>> layer_mfma;
    // per layer, q|k|v and gate|up as one copy each (the linears that share
    // an input in one launch; when every part is a whole number of tiles)
    std::vector<std::array<DecConvMfma, 2>> layer_cat;
    bool cat = false;
    std::vector<std::vector<DecConvMfma>> cnx_up_mfma;
    std::vector<std::array<DecConvMfma, 2>> pw_mfma;
    unsigned *amax = nullptr;  // [amax_slots][kDecMaxSlots]: max |x| of each such convolution's input, cleared per decode
    int amax_slots = 0;
    qtts_decoder_view w{};  // device pointers
    std::vector<qtts_dec_layer_view> layers;
    std::vector<qtts_upsample_view> upsample;
    std::vector<qtts_vocos_block_view> blocks;
    std::vector<std::vector<qtts_vocos_residual_view>> residuals;
    const float **rest_dev = nullptr;  // device array of the rest codebooks
    int *status = nullptr;
    // work buffers, grown on demand
    std::vector<float *> bufs;
    std::vector<size_t> caps;
    uint32_t *codes = nullptr;
    size_t codes_cap = 0;
    float *audio = nullptr;
    size_t audio_cap = 0;
    ~qtts_decoder() {
        for (float *b : bufs) (void)hipFree(b);
        if (codes) (void)hipFree(codes);
        if (audio) (void)hipFree(audio);
    }
};

namespace {

qtts_status dec_up(qtts_ctx *c, Owner &own, const float *src, size_t n, const float **dst, const char *name) {
    float *d = nullptr;
    QTTS_TRY(upload_array(c, own, src, n, &d, name));
    *dst = d;
    return QTTS_OK;
}

// A convolution's weights: [out][in][k] (causal), [in][out][k] (transposed)
// or [ch][k] (depthwise) -- the same element count but for depthwise.
qtts_status dec_conv(qtts_ctx *c, Owner &own, const qtts_conv_view &v, bool depthwise, qtts_conv_view *d,
                     const char *name) {
    if (v.in_channels <= 0 || v.out_channels <= 0 || v.kernel_size <= 0)
        return fail(c, QTTS_ESHAPE, std::string(name) + ": empty convolution");
    *d = v;
    const size_t wn = depthwise ? (size_t)v.out_channels * v.kernel_size
                                : (size_t)v.in_channels * v.out_channels * v.kernel_size;
    QTTS_TRY(dec_up(c, own, v.weight, wn, &d->weight, name));
    return dec_up(c, own, v.bias, (size_t)v.out_channels, &d->bias, name);
}

// The exponent ew that puts max |W| of a host weight array at
// max |W| * 2^ew in [2^14, 2^15) (0 when every weight is zero).
int dec_weight_exponent(const float *w, size_t n) {
    float mx = 0.0f;
    for (size_t i = 0; i < n; i++) {
        const float a = std::fabs(w[i]);
        if (a > mx) mx = a;  // NaN never compares greater
    }
    if (!(mx > 0.0f && std::isfinite(mx))) return 0;
    int E;
    (void)std::frexp(mx, &E);
    return std::min(15 - E, 126);
}

// A matrix-core operand copy (k_dec_conv_repack) of the device weights dw:
// element (m, ci, tap) at dw[m * sm + ci * sci + k0 + tap * kd], scaled by
// 2^ew and split into binary16 hi + lo.
qtts_status dec_mfma_copy(qtts_ctx *c, Owner &own, const float *dw, long long sm, long long sci, int k0, int kd,
                          int M, int cin, int taps, int ew, DecConvMfma *out) {
    DecConvMfma m;
    m.ew = ew;
    m.cin16 = (cin + 15) / 16 * 16;
    m.mtiles = (M + 31) / 32;
    m.ksteps = (taps * m.cin16 / 16 + kConvStage - 1) / kConvStage * kConvStage;
    const size_t n = (size_t)m.mtiles * m.ksteps * 64 * 8;
    QTTS_TRY(own.alloc(c, &m.wh, n));
    QTTS_TRY(own.alloc(c, &m.wl, n));
    launch_dec_conv_repack(c->stream, dw, sm, sci, k0, kd, M, cin, taps, m.cin16, m.mtiles, m.ksteps, ew, m.wh, m.wl);
    QTTS_TRY(check_launch(c, "k_dec_conv_repack"));
    *out = m;
    return QTTS_OK;
}

// A causal convolution's copy (host view h for the weight maximum, device
// view dv for the repack).
qtts_status dec_conv_mfma(qtts_ctx *c, Owner &own, const qtts_conv_view &h, const qtts_conv_view &dv,
                          DecConvMfma *out) {
    const int ci = h.in_channels, co = h.out_channels, k = h.kernel_size;
    const int ew = dec_weight_exponent(h.weight, (size_t)ci * co * k);
    return dec_mfma_copy(c, own, dv.weight, (long long)ci * k, k, 0, 1, co, ci, k, ew, out);
}

// A transposed convolution's copy, one per output phase r: tap t of phase r
// is kernel index r + (J - 1 - t) * stride (J = kernel / stride taps).
qtts_status dec_convt_mfma(qtts_ctx *c, Owner &own, const qtts_conv_view &h, const qtts_conv_view &dv,
                           std::vector<DecConvMfma> *out) {
    const int ci = h.in_channels, co = h.out_channels, k = h.kernel_size, s = h.stride, J = k / s;
    const int ew = dec_weight_exponent(h.weight, (size_t)ci * co * k);
    out->assign((size_t)s, DecConvMfma{});
    for (int r = 0; r < s; r++)
        QTTS_TRY(dec_mfma_copy(c, own, dv.weight, k, (long long)co * k, r + (J - 1) * s, -s, co, ci, J, ew,
                               &(*out)[(size_t)r]));
    return QTTS_OK;
}

// A linear layer's copy: W [K][N] (in-major, as dec_linear reads it), output
// feature m = n of W, channel ci = k.
qtts_status dec_lin_mfma(qtts_ctx *c, Owner &own, const float *hw, const float *dw, int K, int N, DecConvMfma *out) {
    const int ew = dec_weight_exponent(hw, (size_t)K * N);
    return dec_mfma_copy(c, own, dw, 1, N, 0, 0, N, K, 1, ew, out);
}

// Linear layers that read one input, as one copy: part p's N output
// features (a multiple of 32) are tiles p * N / 32 .., so the launch's
// output row holds the parts side by side; one weight exponent for all
// (the one of the largest max |W|).
qtts_status dec_lin_mfma_cat(qtts_ctx *c, Owner &own, const float *const *hw, const float *const *dw, int parts,
                             int K, int N, DecConvMfma *out) {
    int ew = 0;
    for (int q = 0; q < parts; q++) {
        const int e = dec_weight_exponent(hw[q], (size_t)K * N);
        ew = q == 0 ? e : std::min(ew, e);
    }
    DecConvMfma m;
    m.ew = ew;
    m.cin16 = (K + 15) / 16 * 16;
    const int tiles = N / 32;
    m.mtiles = parts * tiles;
    m.ksteps = (m.cin16 / 16 + kConvStage - 1) / kConvStage * kConvStage;
    const size_t per = (size_t)tiles * m.ksteps * 64 * 8;
    QTTS_TRY(own.alloc(c, &m.wh, per * parts));
    QTTS_TRY(own.alloc(c, &m.wl, per * parts));
    for (int q = 0; q < parts; q++) {
        launch_dec_conv_repack(c->stream, dw[q], 1, N, 0, 0, N, K, 1, m.cin16, tiles, m.ksteps, ew, m.wh + per * q,
                               m.wl + per * q);
        QTTS_TRY(check_launch(c, "k_dec_conv_repack"));
    }
    *out = m;
    return QTTS_OK;
}

qtts_status dec_check_transposed(qtts_ctx *c, const qtts_conv_view &v, int in_ch, const char *name) {
    if (v.in_channels != in_ch || v.stride <= 0 || v.padding != 0 || v.kernel_size < v.stride ||
        v.kernel_size % v.stride != 0)
        return fail(c, QTTS_ESHAPE, std::string(name) +
                                        ": transposed convolution needs in_channels to match, padding 0 and a "
                                        "kernel that is a multiple of the stride");
    return QTTS_OK;
}

float *dec_buf(qtts_decoder *d, size_t i, size_t n, qtts_status *st) {
    if (d->bufs.size() <= i) {
        d->bufs.resize(i + 1, nullptr);
        d->caps.resize(i + 1, 0);
    }
    if (d->caps[i] < n) {
        (void)hipStreamSynchronize(d->ctx->stream);
        (void)hipFree(d->bufs[i]);
        d->bufs[i] = nullptr;
        d->caps[i] = 0;
        if (hipMalloc(&d->bufs[i], n * sizeof(float)) != hipSuccess) {
            *st = fail(d->ctx, QTTS_ENOMEM, "decoder work buffer");
            return nullptr;
        }
        d->caps[i] = n;
    }
    return d->bufs[i];
}

int64_t dec_len_after(const qtts_conv_view &v, int64_t len) {
    const int64_t full = (len - 1) * v.stride - 2 * v.padding + v.kernel_size;
    const int64_t crop = v.kernel_size - v.stride;
    return crop > 0 ? full - crop : full;
}

// Causal convolution (causal_conv1d, src/conv.rs:114-184) of x [in][len]
// into c [out][len] on the matrix cores (k_dec_conv_mfma), from the
// weights' binary16 operand copy; xmax: kDecMaxSlots words whose maximum is
// the bits of max |x|.
qtts_status dec_causal_mfma(qtts_decoder *d, const qtts_conv_view &v, const DecConvMfma &m, const float *x,
                            const unsigned *xmax, int len, float *c, int epi, const float *resid = nullptr) {
    DecConvMfmaParams p{};
    p.wh = m.wh;
    p.wl = m.wl;
    p.ew = m.ew;
    p.M = v.out_channels;
    p.mtiles = m.mtiles;
    p.ksteps = m.ksteps;
    p.cin = v.in_channels;
    p.cin16 = m.cin16;
    p.ksize = v.kernel_size;
    p.dilation = v.dilation;
    p.len = len;
    p.x = x;
    p.sxc = len;
    p.sxn = 1;
    p.xmax = xmax;
    p.bias = v.bias;
    p.epi = epi;
    p.c = c;
    p.ldc = len;
    p.out_stride = 1;
    p.phase = 0;
    p.resid = resid;
    launch_dec_conv_mfma(d->ctx->stream, p);
    return check_launch(d->ctx, "k_dec_conv_mfma");
}

// Y(row, n) = X[rows][K] . W[K][N] (+ bias, act) with x(row, k) at
// x[row * sxm + k * sxk] and the output at c[row * scm + n * scn]: the
// transformer's and ConvNeXt's projections, on the matrix cores
// (k_dec_conv_mfma with one tap: output feature n is channel m = n at
// position row).
qtts_status dec_linear_mfma(qtts_decoder *d, const DecConvMfma &m, const float *x, long long sxm, long long sxk,
                            int rows, int K, int N, const unsigned *xmax, const float *bias, float *c, long long scm,
                            long long scn, int epi, const float *scale = nullptr, const float *resid = nullptr,
                            int act = DEC_ACT_NONE) {
    DecConvMfmaParams p{};
    p.wh = m.wh;
    p.wl = m.wl;
    p.ew = m.ew;
    p.M = N;
    p.mtiles = m.mtiles;
    p.ksteps = m.ksteps;
    p.cin = K;
    p.cin16 = m.cin16;
    p.ksize = 1;
    p.dilation = 1;
    p.len = rows;
    p.x = x;
    p.sxc = sxk;
    p.sxn = sxm;
    p.xmax = xmax;
    p.bias = bias;
    p.scale = scale;
    p.act = act;
    p.epi = epi;
    p.c = c;
    p.ldc = scn;
    p.out_stride = scm;
    p.phase = 0;
    p.resid = resid;
    launch_dec_conv_mfma(d->ctx->stream, p);
    return check_launch(d->ctx, "k_dec_conv_mfma");
}

// conv_transpose1d + the causal right crop (src/conv.rs:198-268,
// src/decoder.rs:430-444) on the matrix cores: output phase r
// (out[q * stride + r], q < len) is a causal convolution of x with
// J = kernel / stride taps reaching J - 1 steps back, from the phase's
// operand copy.
qtts_status dec_transposed_mfma(qtts_decoder *d, const qtts_conv_view &v, const std::vector<DecConvMfma> &ph,
                                const float *x, const unsigned *xmax, int len, float *c) {
    const int J = v.kernel_size / v.stride;
    // up to kDecMaxPhases output phases in one launch (grid z = phase): the
    // phases share their input, shapes and weight exponent
    const bool one = v.stride > 1 && v.stride <= kDecMaxPhases;
    for (int r = 0; r < v.stride; r++) {
        const DecConvMfma &m = ph[(size_t)r];
        DecConvMfmaParams p{};
        if (one) {
            p.nphase = v.stride;
            for (int q = 0; q < v.stride; q++) {
                p.ph_wh[q] = ph[(size_t)q].wh;
                p.ph_wl[q] = ph[(size_t)q].wl;
            }
        }
        p.wh = m.wh;
        p.wl = m.wl;
        p.ew = m.ew;
        p.M = v.out_channels;
        p.mtiles = m.mtiles;
        p.ksteps = m.ksteps;
        p.cin = v.in_channels;
        p.cin16 = m.cin16;
        p.ksize = J;
        p.dilation = 1;
        p.len = len;
        p.x = x;
        p.sxc = len;
        p.sxn = 1;
        p.xmax = xmax;
        p.bias = v.bias;
        p.epi = DEC_EPI_STORE;
        p.c = c;
        p.ldc = (long long)len * v.stride;
        p.out_stride = v.stride;
        p.phase = r;
        launch_dec_conv_mfma(d->ctx->stream, p);
        QTTS_TRY(check_launch(d->ctx, "k_dec_conv_mfma"));
        if (one) break;  // the launch ran every phase
    }
    return QTTS_OK;
}

qtts_status dec_decode(qtts_decoder *d, const uint32_t *d_codes, int T, int ld, float *d_audio, int64_t capacity,
                       int64_t *n_samples) {
    qtts_ctx *c = d->ctx;
    const qtts_decoder_view &w = d->w;
    hipStream_t st = c->stream;
    *n_samples = 0;
    if (T <= 0) return QTTS_OK;
    const int64_t need = qtts_decoder_num_samples(d, T);
    if (need > capacity) return fail(c, QTTS_ERANGE, "audio buffer smaller than the decoded length");
    const int cd = w.codebook_dim, vq = w.vq_dim, lat = w.pre_conv.out_channels, hid = w.hidden_size;
    const int ad = w.num_heads * w.head_dim, inter = w.intermediate_size;
    // the largest channel-first signal and ConvNeXt inner activation
    size_t big = std::max((size_t)lat, (size_t)vq) * T, inner_max = 0;
    int64_t len = T;
    for (const auto &u : d->upsample) {
        len = len * u.conv_t.stride;
        big = std::max(big, (size_t)u.channels * len);
        inner_max = std::max(inner_max, (size_t)u.inner_dim * len);
    }
    big = std::max(big, (size_t)w.vocos_init.out_channels * len);
    for (const auto &b : d->blocks) {
        len = len * b.upsample.stride;
        big = std::max(big, (size_t)b.upsample.out_channels * len);
    }
    qtts_status s = QTTS_OK;
    float *S0 = dec_buf(d, 0, big, &s), *S1 = dec_buf(d, 1, big, &s), *S2 = dec_buf(d, 2, big, &s);
    float *S3 = dec_buf(d, 3, big, &s);
    float *E0 = dec_buf(d, 4, (size_t)T * cd, &s), *ES = dec_buf(d, 5, (size_t)T * cd, &s);
    float *X = dec_buf(d, 6, (size_t)T * hid, &s), *XN = dec_buf(d, 7, (size_t)T * hid, &s);
    float *Q = dec_buf(d, 8, (size_t)T * ad, &s), *K = dec_buf(d, 9, (size_t)T * ad, &s);
    float *V = dec_buf(d, 10, (size_t)T * ad, &s), *AO = dec_buf(d, 11, (size_t)T * ad, &s);
    float *G = dec_buf(d, 12, (size_t)T * inter, &s), *U = dec_buf(d, 13, (size_t)T * inter, &s);
    float *P1 = dec_buf(d, 14, std::max<size_t>(inner_max, 1), &s);
    float *QKV = d->cat ? dec_buf(d, 15, (size_t)T * 3 * ad, &s) : nullptr;
    float *GU = d->cat ? dec_buf(d, 16, (size_t)T * 2 * inter, &s) : nullptr;
    if (s != QTTS_OK) return s;

    // Every matrix-core layer scales its input by a power of two from the
    // input's max |x|, gathered into a fresh group of slots (cleared here).
    launch_dec_fill_u32(st, d->amax, d->amax_slots * kDecMaxSlots, 0u);
    QTTS_TRY(check_launch(c, "k_dec_fill_u32"));
    int slot = 0;
    auto take = [&]() -> unsigned * {
        return slot < d->amax_slots ? d->amax + (size_t)(slot++) * kDecMaxSlots : nullptr;
    };
    auto maxof = [&](const float *x, size_t n, unsigned **out) -> qtts_status {
        *out = take();
        if (!*out) return fail(c, QTTS_EDEVICE, "decoder: more matrix-core inputs than max slots");
        launch_dec_absmax(st, x, n, *out);
        return check_launch(c, "k_dec_absmax");
    };
    unsigned *mx = nullptr, *mx2 = nullptr;
    // 1. codebook lookup -> S0 [vq][T] (src/decoder.rs:142-189)
    DecGatherParams g{};
    g.codes = d_codes;
    g.ld = ld;
    g.cd = cd;
    g.cb_size = w.codebook_size;
    g.num_rest = w.num_rest;
    g.first = w.first_codebook;
    g.rest = d->rest_dev;
    g.e0 = E0;
    g.es = ES;
    g.status = d->status;
    launch_dec_gather(st, g, T);
    QTTS_TRY(check_launch(c, "k_dec_gather"));
    QTTS_TRY(maxof(E0, (size_t)T * cd, &mx));
    QTTS_TRY(maxof(ES, (size_t)T * cd, &mx2));
    QTTS_TRY(dec_linear_mfma(d, d->proj0, E0, cd, 1, T, cd, vq, mx, nullptr, S0, 1, T, DEC_EPI_STORE));
    QTTS_TRY(dec_linear_mfma(d, d->proj_rest, ES, cd, 1, T, cd, vq, mx2, nullptr, S0, 1, T, DEC_EPI_ACCUM));
    // 2. pre-conv -> S1 [lat][T]
    QTTS_TRY(maxof(S0, (size_t)vq * T, &mx));
    QTTS_TRY(dec_causal_mfma(d, w.pre_conv, d->pre_conv, S0, mx, T, S1, DEC_EPI_STORE));
    // 3. transformer (src/decoder.rs:195-330) -> S0 [lat][T]
    QTTS_TRY(maxof(S1, (size_t)lat * T, &mx));
    QTTS_TRY(dec_linear_mfma(d, d->tf_in, S1, 1, T, T, lat, hid, mx, w.tf_input_b, X, hid, 1, DEC_EPI_STORE));
    DecAttnParams a{};
    a.q = Q;
    a.k = K;
    a.v = V;
    a.ld = ad;
    a.out = AO;
    a.T = T;
    a.heads = w.num_heads;
    a.hd = w.head_dim;
    a.window = w.sliding_window;
    a.scale = 1.0f / sqrtf((float)w.head_dim);
    for (size_t li = 0; li < d->layers.size(); li++) {
        const qtts_dec_layer_view &L = d->layers[li];
        const std::array<DecConvMfma, 7> &lm = d->layer_mfma[li];
        launch_dec_rmsnorm(st, X, L.input_norm, T, hid, 1e-5f, XN);
        QTTS_TRY(check_launch(c, "k_dec_rmsnorm"));
        QTTS_TRY(maxof(XN, (size_t)T * hid, &mx));
        if (d->cat) {
            // q|k|v in one launch: row t holds q, k, v side by side (3 * ad)
            QTTS_TRY(dec_linear_mfma(d, d->layer_cat[li][0], XN, hid, 1, T, hid, 3 * ad, mx, nullptr, QKV, 3 * ad, 1,
                                     DEC_EPI_STORE));
            a.q = QKV;
            a.k = QKV + ad;
            a.v = QKV + 2 * ad;
            a.ld = 3 * ad;
        } else {
            QTTS_TRY(dec_linear_mfma(d, lm[0], XN, hid, 1, T, hid, ad, mx, nullptr, Q, ad, 1, DEC_EPI_STORE));
            QTTS_TRY(dec_linear_mfma(d, lm[1], XN, hid, 1, T, hid, ad, mx, nullptr, K, ad, 1, DEC_EPI_STORE));
            QTTS_TRY(dec_linear_mfma(d, lm[2], XN, hid, 1, T, hid, ad, mx, nullptr, V, ad, 1, DEC_EPI_STORE));
        }
        launch_dec_rope(st, const_cast<float *>(a.q), const_cast<float *>(a.k), T, w.num_heads, w.head_dim, w.rope_cos,
                        w.rope_sin, w.rope_rows, a.ld);
        QTTS_TRY(check_launch(c, "k_dec_rope"));
        launch_dec_attn(st, a);
        QTTS_TRY(check_launch(c, "k_dec_attn"));
        QTTS_TRY(maxof(AO, (size_t)T * ad, &mx));
        QTTS_TRY(dec_linear_mfma(d, lm[3], AO, ad, 1, T, ad, hid, mx, nullptr, X, hid, 1, DEC_EPI_SCALED_RESID,
                                 L.attn_scale));
        launch_dec_rmsnorm(st, X, L.post_attn_norm, T, hid, 1e-5f, XN);
        QTTS_TRY(check_launch(c, "k_dec_rmsnorm"));
        QTTS_TRY(maxof(XN, (size_t)T * hid, &mx));
        if (d->cat) {
            // gate|up in one launch (row t: gate then up), SiLU(gate) * up into G
            QTTS_TRY(dec_linear_mfma(d, d->layer_cat[li][1], XN, hid, 1, T, hid, 2 * inter, mx, nullptr, GU, 2 * inter,
                                     1, DEC_EPI_STORE));
            launch_dec_swiglu(st, GU, GU + inter, T, inter, 2 * inter, G);
        } else {
            QTTS_TRY(dec_linear_mfma(d, lm[4], XN, hid, 1, T, hid, inter, mx, nullptr, G, inter, 1, DEC_EPI_STORE));
            QTTS_TRY(dec_linear_mfma(d, lm[5], XN, hid, 1, T, hid, inter, mx, nullptr, U, inter, 1, DEC_EPI_STORE));
            launch_dec_swiglu(st, G, U, T, inter, inter, G);
        }
        QTTS_TRY(check_launch(c, "k_dec_swiglu"));
        QTTS_TRY(maxof(G, (size_t)T * inter, &mx));
        QTTS_TRY(dec_linear_mfma(d, lm[6], G, inter, 1, T, inter, hid, mx, nullptr, X, hid, 1, DEC_EPI_SCALED_RESID,
                                 L.mlp_scale));
    }
    launch_dec_rmsnorm(st, X, w.tf_norm, T, hid, 1e-5f, XN);
    QTTS_TRY(check_launch(c, "k_dec_rmsnorm"));
    QTTS_TRY(maxof(XN, (size_t)T * hid, &mx));
    QTTS_TRY(dec_linear_mfma(d, d->tf_out, XN, hid, 1, T, hid, lat, mx, w.tf_output_b, S0, 1, T, DEC_EPI_STORE));
    // 4. upsample: transposed conv + ConvNeXt (src/decoder.rs:336-388, 424-448)
    float *const pool[4] = {S0, S1, S2, S3};
    auto other = [&](const float *a, const float *b = nullptr, const float *c3 = nullptr) {
        for (float *p : pool)
            if (p != a && p != b && p != c3) return p;
        return (float *)nullptr;
    };
    float *sig = S0;
    int L = T;
    for (size_t ui = 0; ui < d->upsample.size(); ui++) {
        const qtts_upsample_view &u = d->upsample[ui];
        float *up = other(sig), *dw = other(sig, up), *nrm = other(sig, up, dw);
        QTTS_TRY(maxof(sig, (size_t)u.channels * L, &mx));
        QTTS_TRY(dec_transposed_mfma(d, u.conv_t, d->cnx_up_mfma[ui], sig, mx, L, up));
        L *= u.conv_t.stride;
        launch_dec_dwconv(st, up, u.dw_conv.weight, u.dw_conv.bias, u.channels, L, u.dw_conv.kernel_size, dw);
        QTTS_TRY(check_launch(c, "k_dec_dwconv"));
        launch_dec_lnorm(st, dw, u.norm_w, u.norm_b, u.channels, L, 1e-5f, nrm);
        QTTS_TRY(check_launch(c, "k_dec_lnorm"));
        QTTS_TRY(maxof(nrm, (size_t)u.channels * L, &mx));
        QTTS_TRY(dec_linear_mfma(d, d->pw_mfma[ui][0], nrm, 1, L, L, u.channels, u.inner_dim, mx, u.pw1_b, P1,
                                 u.inner_dim, 1, DEC_EPI_STORE, nullptr, nullptr, DEC_ACT_GELU));
        // out = residual + gamma * pw2 (the residual is the stage input `up`)
        QTTS_TRY(maxof(P1, (size_t)L * u.inner_dim, &mx));
        QTTS_TRY(dec_linear_mfma(d, d->pw_mfma[ui][1], P1, u.inner_dim, 1, L, u.inner_dim, u.channels, mx, u.pw2_b,
                                 dw, 1, L, DEC_EPI_RESID_IN, u.gamma, up));
        sig = dw;
    }
    // 5. Vocos (src/decoder.rs:450-495)
    {
        float *o = other(sig);
        QTTS_TRY(maxof(sig, (size_t)w.vocos_init.in_channels * L, &mx));
        QTTS_TRY(dec_causal_mfma(d, w.vocos_init, d->vocos_init, sig, mx, L, o, DEC_EPI_STORE));
        sig = o;
    }
    // a residual unit's conv2 output still to be added to sig: the SnakeBeta
    // that next reads sig adds it and stores the sum (faster than the conv2
    // epilogue reading each residual), the same f32 addition
    float *pend = nullptr;
    for (size_t bi = 0; bi < d->blocks.size(); bi++) {
        const qtts_vocos_block_view &b = d->blocks[bi];
        const int cin = b.upsample.in_channels, cout = b.upsample.out_channels;
        float *t1 = other(sig), *nxt = other(sig, t1);
        unsigned *m0 = take();
        if (!m0) return fail(c, QTTS_EDEVICE, "decoder: more matrix-core inputs than max slots");
        launch_dec_snake(st, sig, b.pre_snake_alpha, b.pre_snake_beta, cin, L, t1, m0, pend, pend ? sig : nullptr);
        pend = nullptr;
        QTTS_TRY(check_launch(c, "k_dec_snake"));
        QTTS_TRY(dec_transposed_mfma(d, b.upsample, d->up_mfma[bi], t1, m0, L, nxt));
        L *= b.upsample.stride;
        sig = nxt;
        float *t2 = other(sig, t1);
        for (int r = 0; r < b.num_residuals; r++) {
            const qtts_vocos_residual_view &rv = b.residuals[r];
            const std::array<DecConvMfma, 2> &mc = d->res_mfma[bi][(size_t)r];
            unsigned *m1 = take(), *m2 = take();
            if (!m1 || !m2) return fail(c, QTTS_EDEVICE, "decoder: more matrix-core inputs than max slots");
            launch_dec_snake(st, sig, rv.act1_alpha, rv.act1_beta, cout, L, t1, m1, pend, pend ? sig : nullptr);
            pend = nullptr;
            QTTS_TRY(check_launch(c, "k_dec_snake"));
            QTTS_TRY(dec_causal_mfma(d, rv.conv1, mc[0], t1, m1, L, t2, DEC_EPI_STORE));
            launch_dec_snake(st, t2, rv.act2_alpha, rv.act2_beta, cout, L, t1, m2);
            QTTS_TRY(check_launch(c, "k_dec_snake"));
            // signal = residual + conv2: conv2 into t2, added by the next SnakeBeta
            QTTS_TRY(dec_causal_mfma(d, rv.conv2, mc[1], t1, m2, L, t2, DEC_EPI_STORE));
            pend = t2;
        }
    }
    float *t1 = other(sig);
    // 6. final SnakeBeta, output conv, clamp to [-1, 1]
    unsigned *mf = take();
    if (!mf) return fail(c, QTTS_EDEVICE, "decoder: more matrix-core inputs than max slots");
    launch_dec_snake(st, sig, w.final_snake_alpha, w.final_snake_beta, w.output_conv.in_channels, L, t1, mf, pend,
                     pend ? sig : nullptr);
    QTTS_TRY(check_launch(c, "k_dec_snake"));
    QTTS_TRY(dec_causal_mfma(d, w.output_conv, d->out_conv, t1, mf, L, d_audio, DEC_EPI_CLAMP));
    *n_samples = (int64_t)L * w.output_conv.out_channels;
    return QTTS_OK;
}

}  // namespace

extern "C" {

qtts_status qtts_decoder_upload(qtts_ctx *c, const qtts_decoder_view *v, qtts_decoder **out) {
    if (!c || !v || !out) return QTTS_EINVAL;
    *out = nullptr;
    qtts_decoder *d = new qtts_decoder();
    d->ctx = ctx_retain(c);
    auto bail = [&](qtts_status s) {
        delete d;
        ctx_release(c);
        return s;
    };
    Owner &o = d->own;
    qtts_decoder_view &w = d->w;
    w = *v;
    const int cd = v->codebook_dim, vq = v->vq_dim, hid = v->hidden_size, ad = v->num_heads * v->head_dim;
    const int inter = v->intermediate_size, lat = v->pre_conv.out_channels;
    if (cd <= 0 || vq <= 0 || hid <= 0 || v->num_heads <= 0 || v->head_dim <= 0 || v->head_dim % 2 || inter <= 0 ||
        v->codebook_size <= 0 || v->num_rest < 0 || v->sliding_window <= 0 || v->num_layers < 0 ||
        v->rope_rows < 0)
        return bail(fail(c, QTTS_ESHAPE, "decoder: bad configuration"));
    if (v->head_dim > kDecMaxHeadDim || v->sliding_window > kDecMaxWindow)
        return bail(fail(c, QTTS_ESHAPE, "decoder: head_dim or sliding_window above the attention kernel's limit"));
    if (v->pre_conv.in_channels != vq) return bail(fail(c, QTTS_ESHAPE, "decoder: pre_conv input != vq_dim"));
    qtts_status s;
    auto up = [&](const float *src, size_t n, const float **dst, const char *name) {
        return dec_up(c, o, src, n, dst, name);
    };
    const size_t cbn = (size_t)v->codebook_size * cd;
    if ((s = up(v->first_codebook, cbn, &w.first_codebook, "first_codebook")) != QTTS_OK ||
        (s = up(v->first_output_proj, (size_t)cd * vq, &w.first_output_proj, "first_output_proj")) != QTTS_OK ||
        (s = up(v->rest_output_proj, (size_t)cd * vq, &w.rest_output_proj, "rest_output_proj")) != QTTS_OK)
        return bail(s);
    if ((s = dec_lin_mfma(c, o, v->first_output_proj, w.first_output_proj, cd, vq, &d->proj0)) != QTTS_OK ||
        (s = dec_lin_mfma(c, o, v->rest_output_proj, w.rest_output_proj, cd, vq, &d->proj_rest)) != QTTS_OK)
        return bail(s);
    std::vector<const float *> rest((size_t)std::max(v->num_rest, 1), nullptr);
    for (int g = 0; g < v->num_rest; g++)
        if (!v->rest_codebooks || (s = up(v->rest_codebooks[g], cbn, &rest[g], "rest_codebook")) != QTTS_OK)
            return bail(s != QTTS_OK ? s : fail(c, QTTS_EINVAL, "rest_codebooks: null"));
    if ((s = o.alloc(c, &d->rest_dev, rest.size())) != QTTS_OK) return bail(s);
    if (hipMemcpy(d->rest_dev, rest.data(), rest.size() * sizeof(float *), hipMemcpyHostToDevice) != hipSuccess)
        return bail(fail(c, QTTS_EDEVICE, "hipMemcpy"));
    w.rest_codebooks = nullptr;
    if ((s = dec_conv(c, o, v->pre_conv, false, &w.pre_conv, "pre_conv")) != QTTS_OK ||
        (s = dec_conv_mfma(c, o, v->pre_conv, w.pre_conv, &d->pre_conv)) != QTTS_OK)
        return bail(s);
    if ((s = up(v->tf_input_w, (size_t)lat * hid, &w.tf_input_w, "tf_input_w")) != QTTS_OK ||
        (s = up(v->tf_input_b, (size_t)hid, &w.tf_input_b, "tf_input_b")) != QTTS_OK ||
        (s = up(v->tf_norm, (size_t)hid, &w.tf_norm, "tf_norm")) != QTTS_OK ||
        (s = up(v->tf_output_w, (size_t)hid * lat, &w.tf_output_w, "tf_output_w")) != QTTS_OK ||
        (s = up(v->tf_output_b, (size_t)lat, &w.tf_output_b, "tf_output_b")) != QTTS_OK ||
        (s = dec_lin_mfma(c, o, v->tf_input_w, w.tf_input_w, lat, hid, &d->tf_in)) != QTTS_OK ||
        (s = dec_lin_mfma(c, o, v->tf_output_w, w.tf_output_w, hid, lat, &d->tf_out)) != QTTS_OK)
        return bail(s);
    for (int l = 0; l < v->num_layers; l++) {
        const qtts_dec_layer_view &L = v->layers[l];
        qtts_dec_layer_view D{};
        if ((s = up(L.q_proj, (size_t)hid * ad, &D.q_proj, "q_proj")) != QTTS_OK ||
            (s = up(L.k_proj, (size_t)hid * ad, &D.k_proj, "k_proj")) != QTTS_OK ||
            (s = up(L.v_proj, (size_t)hid * ad, &D.v_proj, "v_proj")) != QTTS_OK ||
            (s = up(L.o_proj, (size_t)ad * hid, &D.o_proj, "o_proj")) != QTTS_OK ||
            (s = up(L.gate_proj, (size_t)hid * inter, &D.gate_proj, "gate_proj")) != QTTS_OK ||
            (s = up(L.up_proj, (size_t)hid * inter, &D.up_proj, "up_proj")) != QTTS_OK ||
            (s = up(L.down_proj, (size_t)inter * hid, &D.down_proj, "down_proj")) != QTTS_OK ||
            (s = up(L.input_norm, (size_t)hid, &D.input_norm, "input_norm")) != QTTS_OK ||
            (s = up(L.post_attn_norm, (size_t)hid, &D.post_attn_norm, "post_attn_norm")) != QTTS_OK ||
            (s = up(L.attn_scale, (size_t)hid, &D.attn_scale, "attn_scale")) != QTTS_OK ||
            (s = up(L.mlp_scale, (size_t)hid, &D.mlp_scale, "mlp_scale")) != QTTS_OK)
            return bail(s);
        std::array<DecConvMfma, 7> lm{};
        if ((s = dec_lin_mfma(c, o, L.q_proj, D.q_proj, hid, ad, &lm[0])) != QTTS_OK ||
            (s = dec_lin_mfma(c, o, L.k_proj, D.k_proj, hid, ad, &lm[1])) != QTTS_OK ||
            (s = dec_lin_mfma(c, o, L.v_proj, D.v_proj, hid, ad, &lm[2])) != QTTS_OK ||
            (s = dec_lin_mfma(c, o, L.o_proj, D.o_proj, ad, hid, &lm[3])) != QTTS_OK ||
            (s = dec_lin_mfma(c, o, L.gate_proj, D.gate_proj, hid, inter, &lm[4])) != QTTS_OK ||
            (s = dec_lin_mfma(c, o, L.up_proj, D.up_proj, hid, inter, &lm[5])) != QTTS_OK ||
            (s = dec_lin_mfma(c, o, L.down_proj, D.down_proj, inter, hid, &lm[6])) != QTTS_OK)
            return bail(s);
        d->layer_mfma.push_back(lm);
        d->cat = ad % 32 == 0 && inter % 32 == 0;
        if (d->cat) {
            std::array<DecConvMfma, 2> lc{};
            const float *hq[3] = {L.q_proj, L.k_proj, L.v_proj}, *dq[3] = {D.q_proj, D.k_proj, D.v_proj};
            const float *hg[2] = {L.gate_proj, L.up_proj}, *dg[2] = {D.gate_proj, D.up_proj};
            if ((s = dec_lin_mfma_cat(c, o, hq, dq, 3, hid, ad, &lc[0])) != QTTS_OK ||
                (s = dec_lin_mfma_cat(c, o, hg, dg, 2, hid, inter, &lc[1])) != QTTS_OK)
                return bail(s);
            d->layer_cat.push_back(lc);
        }
        d->amax_slots += 4;  // the normed rows twice, the attention output, SiLU(gate) * up
        d->layers.push_back(D);
    }
    w.layers = nullptr;
    int ch = lat;
    for (int i = 0; i < v->num_upsample; i++) {
        const qtts_upsample_view &U = v->upsample[i];
        qtts_upsample_view D = U;
        if (U.channels != ch || U.conv_t.out_channels != ch || U.dw_conv.out_channels != ch || U.inner_dim <= 0)
            return bail(fail(c, QTTS_ESHAPE, "decoder: upsample stage channels do not chain"));
        if ((s = dec_check_transposed(c, U.conv_t, ch, "upsample conv_t")) != QTTS_OK) return bail(s);
        if ((s = dec_conv(c, o, U.conv_t, false, &D.conv_t, "upsample conv_t")) != QTTS_OK ||
            (s = dec_conv(c, o, U.dw_conv, true, &D.dw_conv, "upsample dw_conv")) != QTTS_OK ||
            (s = up(U.norm_w, (size_t)ch, &D.norm_w, "norm_w")) != QTTS_OK ||
            (s = up(U.norm_b, (size_t)ch, &D.norm_b, "norm_b")) != QTTS_OK ||
            (s = up(U.pw1_w, (size_t)ch * U.inner_dim, &D.pw1_w, "pw1_w")) != QTTS_OK ||
            (s = up(U.pw1_b, (size_t)U.inner_dim, &D.pw1_b, "pw1_b")) != QTTS_OK ||
            (s = up(U.pw2_w, (size_t)U.inner_dim * ch, &D.pw2_w, "pw2_w")) != QTTS_OK ||
            (s = up(U.pw2_b, (size_t)ch, &D.pw2_b, "pw2_b")) != QTTS_OK ||
            (s = up(U.gamma, (size_t)ch, &D.gamma, "gamma")) != QTTS_OK)
            return bail(s);
        std::vector<DecConvMfma> ph;
        std::array<DecConvMfma, 2> pw{};
        if ((s = dec_convt_mfma(c, o, U.conv_t, D.conv_t, &ph)) != QTTS_OK ||
            (s = dec_lin_mfma(c, o, U.pw1_w, D.pw1_w, ch, U.inner_dim, &pw[0])) != QTTS_OK ||
            (s = dec_lin_mfma(c, o, U.pw2_w, D.pw2_w, U.inner_dim, ch, &pw[1])) != QTTS_OK)
            return bail(s);
        d->cnx_up_mfma.push_back(ph);
        d->pw_mfma.push_back(pw);
        d->amax_slots += 3;  // the stage input, the LayerNorm output, GELU(pw1)
        d->upsample.push_back(D);
    }
    w.upsample = nullptr;
    if (v->vocos_init.in_channels != ch) return bail(fail(c, QTTS_ESHAPE, "decoder: vocos_init input channels"));
    if ((s = dec_conv(c, o, v->vocos_init, false, &w.vocos_init, "vocos_init")) != QTTS_OK ||
        (s = dec_conv_mfma(c, o, v->vocos_init, w.vocos_init, &d->vocos_init)) != QTTS_OK)
        return bail(s);
    ch = v->vocos_init.out_channels;
    d->residuals.resize((size_t)std::max(v->num_vocos_blocks, 0));
    d->res_mfma.resize(d->residuals.size());
    d->up_mfma.resize(d->residuals.size());
    for (int b = 0; b < v->num_vocos_blocks; b++) {
        const qtts_vocos_block_view &B = v->vocos_blocks[b];
        qtts_vocos_block_view D = B;
        if ((s = dec_check_transposed(c, B.upsample, ch, "vocos upsample")) != QTTS_OK) return bail(s);
        if ((s = up(B.pre_snake_alpha, (size_t)ch, &D.pre_snake_alpha, "pre_snake_alpha")) != QTTS_OK ||
            (s = up(B.pre_snake_beta, (size_t)ch, &D.pre_snake_beta, "pre_snake_beta")) != QTTS_OK ||
            (s = dec_conv(c, o, B.upsample, false, &D.upsample, "vocos upsample")) != QTTS_OK ||
            (s = dec_convt_mfma(c, o, B.upsample, D.upsample, &d->up_mfma[(size_t)b])) != QTTS_OK)
            return bail(s);
        d->amax_slots += 1;
        ch = B.upsample.out_channels;
        for (int r = 0; r < B.num_residuals; r++) {
            const qtts_vocos_residual_view &R = B.residuals[r];
            qtts_vocos_residual_view E = R;
            if (R.conv1.in_channels != ch || R.conv1.out_channels != ch || R.conv2.in_channels != ch ||
                R.conv2.out_channels != ch)
                return bail(fail(c, QTTS_ESHAPE, "decoder: residual convolutions must keep the channels"));
            if ((s = up(R.act1_alpha, (size_t)ch, &E.act1_alpha, "act1_alpha")) != QTTS_OK ||
                (s = up(R.act1_beta, (size_t)ch, &E.act1_beta, "act1_beta")) != QTTS_OK ||
                (s = up(R.act2_alpha, (size_t)ch, &E.act2_alpha, "act2_alpha")) != QTTS_OK ||
                (s = up(R.act2_beta, (size_t)ch, &E.act2_beta, "act2_beta")) != QTTS_OK ||
                (s = dec_conv(c, o, R.conv1, false, &E.conv1, "residual conv1")) != QTTS_OK ||
                (s = dec_conv(c, o, R.conv2, false, &E.conv2, "residual conv2")) != QTTS_OK)
                return bail(s);
            std::array<DecConvMfma, 2> mc{};
            if ((s = dec_conv_mfma(c, o, R.conv1, E.conv1, &mc[0])) != QTTS_OK ||
                (s = dec_conv_mfma(c, o, R.conv2, E.conv2, &mc[1])) != QTTS_OK)
                return bail(s);
            d->res_mfma[b].push_back(mc);
            d->amax_slots += 2;
            d->residuals[b].push_back(E);
        }
        D.residuals = d->residuals[b].data();
        d->blocks.push_back(D);
    }
    w.vocos_blocks = nullptr;
    if (v->output_conv.in_channels != ch) return bail(fail(c, QTTS_ESHAPE, "decoder: output_conv input channels"));
    if ((s = up(v->final_snake_alpha, (size_t)ch, &w.final_snake_alpha, "final_snake_alpha")) != QTTS_OK ||
        (s = up(v->final_snake_beta, (size_t)ch, &w.final_snake_beta, "final_snake_beta")) != QTTS_OK ||
        (s = dec_conv(c, o, v->output_conv, false, &w.output_conv, "output_conv")) != QTTS_OK ||
        (s = dec_conv_mfma(c, o, v->output_conv, w.output_conv, &d->out_conv)) != QTTS_OK)
        return bail(s);
    // the codebook rows (two), the pre-conv input and output, the
    // transformer's output rows, the Vocos input and the final SnakeBeta
    d->amax_slots += 7;
    const size_t rn = (size_t)v->rope_rows * (v->head_dim / 2);
    if (rn) {
        if ((s = up(v->rope_cos, rn, &w.rope_cos, "rope_cos")) != QTTS_OK ||
            (s = up(v->rope_sin, rn, &w.rope_sin, "rope_sin")) != QTTS_OK)
            return bail(s);
    }
    if ((s = o.alloc(c, &d->status, 1)) != QTTS_OK) return bail(s);
    if (hipMemset(d->status, 0, sizeof(int)) != hipSuccess) return bail(fail(c, QTTS_EDEVICE, "hipMemset"));
    if ((s = o.alloc(c, &d->amax, (size_t)std::max(d->amax_slots, 1) * kDecMaxSlots)) != QTTS_OK) return bail(s);
    if (hipStreamSynchronize(c->stream) != hipSuccess) return bail(fail(c, QTTS_EDEVICE, "decoder weight repack"));
    *out = d;
    return QTTS_OK;
}

void qtts_decoder_free(qtts_decoder *d) {
    if (!d) return;
    qtts_ctx *c = d->ctx;
    if (c) (void)hipStreamSynchronize(c->stream);
    delete d;
    if (c) ctx_release(c);
}

int64_t qtts_decoder_num_samples(const qtts_decoder *d, int32_t frames) {
    if (!d || frames <= 0) return 0;
    int64_t len = frames;
    for (const auto &u : d->upsample) len = dec_len_after(u.conv_t, len);
    for (const auto &b : d->blocks) len = dec_len_after(b.upsample, len);
    return len * d->w.output_conv.out_channels;
}

qtts_status qtts_decode_to_audio_device(qtts_decoder *d, const uint32_t *d_codes, int32_t frames, int32_t ld,
                                        float *d_audio, int64_t capacity, int64_t *n_samples) {
    if (!d || !n_samples || (frames > 0 && (!d_codes || !d_audio || ld < frames))) return QTTS_EINVAL;
    return dec_decode(d, d_codes, frames, ld, d_audio, capacity, n_samples);
}

qtts_status qtts_decode_to_audio(qtts_decoder *d, const uint32_t *codes, int32_t frames, int32_t ld, float *audio,
                                 int64_t capacity, int64_t *n_samples) {
    if (!d || !n_samples || (frames > 0 && (!codes || !audio || ld < frames))) return QTTS_EINVAL;
    qtts_ctx *c = d->ctx;
    *n_samples = 0;
    if (frames <= 0) return QTTS_OK;
    const int groups = d->w.num_rest + 1;
    for (int g = 0; g < groups; g++)
        for (int t = 0; t < frames; t++)
            if (codes[(size_t)g * ld + t] >= (uint32_t)d->w.codebook_size)
                return fail(c, QTTS_ERANGE, "code beyond the codebook");
    const int64_t need = qtts_decoder_num_samples(d, frames);
    if (need > capacity) return fail(c, QTTS_ERANGE, "audio buffer smaller than the decoded length");
    const size_t ncodes = (size_t)groups * frames;
    if (d->codes_cap < ncodes) {
        (void)hipFree(d->codes);
        d->codes = nullptr;
        d->codes_cap = 0;
        HIP_TRY(c, hipMalloc(&d->codes, ncodes * sizeof(uint32_t)));
        d->codes_cap = ncodes;
    }
    if (d->audio_cap < (size_t)need) {
        (void)hipFree(d->audio);
        d->audio = nullptr;
        d->audio_cap = 0;
        HIP_TRY(c, hipMalloc(&d->audio, (size_t)need * sizeof(float)));
        d->audio_cap = (size_t)need;
    }
    for (int g = 0; g < groups; g++)
        HIP_TRY(c, hipMemcpyAsync(d->codes + (size_t)g * frames, codes + (size_t)g * ld, frames * sizeof(uint32_t),
                                  hipMemcpyHostToDevice, c->stream));
    QTTS_TRY(dec_decode(d, d->codes, frames, frames, d->audio, need, n_samples));
    HIP_TRY(c, hipMemcpyAsync(audio, d->audio, (size_t)*n_samples * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

qtts_status qtts_generate_speech(qtts_talker *t, qtts_predictor *p, qtts_decoder *d, const uint32_t *text_tokens,
                                 int32_t n_text, uint32_t speaker_id, uint32_t language_id,
                                 const float *voice_embedding, qtts_kv *talker_kv, qtts_kv *predictor_kv,
                                 const qtts_loop_params *params, uint64_t seed, float *audio, int64_t capacity,
                                 int64_t *n_samples, int32_t *n_frames) {
    if (!t || !d || !params || !n_samples || !n_frames) return QTTS_EINVAL;
    *n_samples = 0;
    *n_frames = 0;
    qtts_ctx *c = t->ctx, *dc = d->ctx;
    if (dc->device != c->device) return fail(c, QTTS_EINVAL, "the decoder is on another device than the talker");
    if (d->w.num_rest + 1 > 16) return fail(c, QTTS_ESHAPE, "the decoder reads more than a frame's 16 code groups");
    const int max_codes = params->max_codes > 0 ? params->max_codes : 0;
    const int64_t most = qtts_decoder_num_samples(d, max_codes);
    if (most > 0 && !audio) return QTTS_EINVAL;
    if (most > capacity) return fail(c, QTTS_ERANGE, "audio buffer smaller than max_codes frames decode to");
    int32_t nf = 0;
    QTTS_TRY(speech_codes(t, p, text_tokens, n_text, speaker_id, language_id, voice_embedding, talker_kv, predictor_kv,
                          params, seed, nullptr, &nf));
    *n_frames = nf;
    if (nf == 0) return QTTS_OK;
    // decode_to_audio (src/generate_new.rs:304-306) of the codes where the
    // frame loop left them: t->codes, [16][max_codes], complete (the loop
    // ends with its stream synchronised).
    const int64_t need = qtts_decoder_num_samples(d, nf);
    if (d->audio_cap < (size_t)need) {
        (void)hipFree(d->audio);
        d->audio = nullptr;
        d->audio_cap = 0;
        HIP_TRY(dc, hipMalloc(&d->audio, (size_t)need * sizeof(float)));
        d->audio_cap = (size_t)need;
    }
    HIP_TRY(dc, hipMemsetAsync(d->status, 0, sizeof(int), dc->stream));
    int64_t n = 0;
    QTTS_TRY(dec_decode(d, t->codes, nf, max_codes, d->audio, need, &n));
    int bad = 0;
    HIP_TRY(dc, hipMemcpyAsync(&bad, d->status, sizeof(int), hipMemcpyDeviceToHost, dc->stream));
    HIP_TRY(dc, hipMemcpyAsync(audio, d->audio, (size_t)n * sizeof(float), hipMemcpyDeviceToHost, dc->stream));
    QTTS_TRY(sync(dc));
    // a semantic code past the decoder's codebook: the reference's lookup
    // (src/decoder.rs:151-152) would index past the table and panic
    if (bad) return fail(c, QTTS_ERANGE, "a generated code is beyond the decoder's codebook");
    *n_samples = n;
    return QTTS_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Batched streams: `batch` independent generate_speech loops
// (src/generate_new.rs:242-300) in lockstep over shared weights.  Every
// product runs on the matrix cores with one row per stream (two per stream
// in the predictor's first pass); attention and the K/V appends address each
// row's own cache through per-row tables.
// ---------------------------------------------------------------------------
namespace {

struct RowTab {
    const float *const *k = nullptr, *const *v = nullptr;  // per-row layer-0 cache bases
    const int *pos = nullptr, *kv = nullptr;               // per-row position / cache row (null: 0)
    int stride = 1, pos0 = 0, kv0 = 0, cap = 0;
};

qtts_status make_stack_mfma(qtts_ctx *c, Owner &own, const Stack &st, std::vector<DevQ4Mfma> *out, bool *ok) {
    std::vector<void *> mems;
    *ok = true;
    for (const DevLayer &Ly : st.L)
        for (const DevQ4 *w : {&Ly.qkv, &Ly.o, &Ly.gu, &Ly.down}) {
            DevQ4Mfma m{};
            void *mem = nullptr;
            bool one = false;
            const qtts_status s = make_mfma_copy(c, *w, &mem, &m, &one);
            if (s != QTTS_OK || !one) {
                for (void *p : mems) (void)hipFree(p);
                out->clear();
                *ok = false;
                return s;
            }
            mems.push_back(mem);
            out->push_back(m);
        }
    for (void *p : mems) own.ptrs.push_back(p);
    return QTTS_OK;
}

qtts_status make_head_mfma(qtts_talker *t) {
    if (t->head_mfma_state != 0) return QTTS_OK;
    void *mem = nullptr;
    bool ok = false;
    QTTS_TRY(make_mfma_copy(t->ctx, t->head, &mem, &t->head_mfma, &ok));
    if (mem) t->own.ptrs.push_back(mem);
    t->head_mfma_state = ok ? 1 : -1;
    return QTTS_OK;
}

qtts_status make_predictor_mfma(qtts_predictor *p) {
    qtts_ctx *c = p->ctx;
    bool ok = false;
    QTTS_TRY(make_stack_mfma(c, p->own, p->st, &p->mfma, &ok));
    std::vector<void *> mems;
    auto one = [&](const DevQ4 &w, DevQ4Mfma *m) -> qtts_status {
        void *mem = nullptr;
        bool good = false;
        QTTS_TRY(make_mfma_copy(c, w, &mem, m, &good));
        if (!good) ok = false;
        if (mem) mems.push_back(mem);
        return QTTS_OK;
    };
    if (ok && !p->identity_proj) QTTS_TRY(one(p->in_proj, &p->mfma_in));
    p->mfma_heads.assign((size_t)p->groups, DevQ4Mfma{});
    for (int g = 0; ok && g < p->groups; g++) QTTS_TRY(one(p->heads[g], &p->mfma_heads[(size_t)g]));
    for (void *m : mems) p->own.ptrs.push_back(m);
    p->mfma_state = ok ? 1 : -1;
    return QTTS_OK;
}

// One layer stack over M independent rows (per-row caches from R).
// fused: every row is its stream's only new row, so the attention kernel
// does k_qkv_rows' work itself (no row attends to another row's new K/V).
qtts_status layers_batched(qtts_ctx *c, const Stack &st, const DevQ4Mfma *W, const RowTab &R, float *x, int M,
                           float *raw, float *q, float *a, int nsplit, bool fused) {
    const int hidden = st.hidden, qd = st.nq * st.hd, nqkv = qd + 2 * st.nkv * st.hd;
    if ((size_t)M * st.nq * nsplit * (st.hd + 2) > kAttnPartFloats || M * st.nkv > kAttnCounters)
        return fail(c, QTTS_ESHAPE, "batched attention: too many rows for the split buffers");
    if (!attn_split_fits(R.cap, nsplit)) return fail(c, QTTS_ESHAPE, "batched attention: a split exceeds the score buffer");
    for (int l = 0; l < st.layers; l++) {
        const DevLayer &Ly = st.L[l];
        const DevQ4Mfma *Wl = W + (size_t)4 * l;
        const long long layer_off = (long long)l * st.nkv * R.cap * st.hd;
        QTTS_TRY(run_gemm_mfma(c, Wl[0], x, M, hidden, MFMA_ROWS_RMSNORM, Ly.in_g, raw, nqkv, nullptr, false));
        QkvRowsParams qp{};
        qp.raw = raw;
        qp.ldr = nqkv;
        qp.M = M;
        qp.n_q_heads = st.nq;
        qp.n_kv_heads = st.nkv;
        qp.head_dim = st.hd;
        qp.q_norm = Ly.q_norm;
        qp.k_norm = Ly.k_norm;
        qp.rope_cos = st.rope_cos;
        qp.rope_sin = st.rope_sin;
        qp.rope_rows = st.rope_rows;
        qp.rope_skip_oob = st.rope_skip_oob;
        qp.q = q;
        qp.ldq = qd;
        qp.kv_cap = R.cap;
        qp.pos0 = R.pos0;
        qp.row0 = R.kv0;
        qp.row_k = R.k;
        qp.row_v = R.v;
        qp.row_pos = R.pos;
        qp.row_kv = R.kv;
        qp.row_stride = R.stride;
        qp.layer_off = layer_off;
        if (!fused) {
            launch_qkv_rows(c->stream, qp);
            QTTS_TRY(check_launch(c, "k_qkv_rows"));
        }
        AttnParams ap{};
        ap.q = q;
        ap.ldq = qd;
        ap.kv_cap = R.cap;
        ap.nq = st.nq;
        ap.nkv = st.nkv;
        ap.hd = st.hd;
        ap.kvlen_const = R.kv0;
        ap.nsplit = nsplit;
        ap.scale = 1.0f / sqrtf((float)st.hd);  // src/talker.rs:305
        ap.part = c->attn_part;
        ap.counters = c->attn_counters;
        ap.out = a;
        ap.ldo = qd;
        ap.row_k = R.k;
        ap.row_v = R.v;
        ap.row_kv = R.kv;
        ap.row_stride = R.stride;
        ap.layer_off = layer_off;
        if (fused) {
            ap.raw = raw;
            ap.ldr = nqkv;
            ap.q_norm = Ly.q_norm;
            ap.k_norm = Ly.k_norm;
            ap.rope_cos = st.rope_cos;
            ap.rope_sin = st.rope_sin;
            ap.rope_rows = st.rope_rows;
            ap.rope_skip_oob = st.rope_skip_oob;
            ap.row_pos = R.pos;
            ap.pos0 = R.pos0;
        }
        launch_attention(c->stream, ap, M);
        QTTS_TRY(check_launch(c, "k_attn"));
        QTTS_TRY(run_gemm_mfma(c, Wl[1], a, M, qd, MFMA_ROWS_PLAIN, nullptr, x, hidden, nullptr, true));
        QTTS_TRY(run_gemm_mfma(c, Wl[2], x, M, hidden, MFMA_ROWS_RMSNORM, Ly.post_g, raw, 2 * st.inter, nullptr,
                               false));
        QTTS_TRY(run_gemm_mfma(c, Wl[3], raw, M, 2 * st.inter, MFMA_ROWS_SWIGLU, nullptr, x, hidden, nullptr, true));
    }
    return QTTS_OK;
}

// Device allocations of one batched call, freed on every return path.
struct DevAllocs {
    std::vector<void *> ptrs;
    ~DevAllocs() {
        for (void *p : ptrs) (void)hipFree(p);
    }
    template <class T>
    qtts_status get(qtts_ctx *c, T **out, size_t count) {
        void *p = nullptr;
        if (hipMalloc(&p, (count ? count : 1) * sizeof(T)) != hipSuccess)
            return fail(c, QTTS_ENOMEM, "batched loop buffers");
        ptrs.push_back(p);
        *out = reinterpret_cast<T *>(p);
        return QTTS_OK;
    }
};

}  // namespace

extern "C" {

qtts_status qtts_generate_codes_batch(qtts_talker *t, qtts_predictor *p, int32_t batch, qtts_kv *const *talker_kvs,
                                      const float *last_hidden, const float *logits, const int32_t *positions,
                                      const float *trailing_text, int32_t trailing_len, const float *tts_pad_embed,
                                      const qtts_loop_params *params, const uint64_t *seeds, uint32_t *codes,
                                      int32_t *n_frames) {
    if (!t || batch < 1 || !talker_kvs || !last_hidden || !logits || !positions || !params || !seeds || !codes ||
        !n_frames)
        return QTTS_EINVAL;
    qtts_ctx *c = t->ctx;
    const bool talker_only = params->talker_only || !p;
    if (!talker_only && (!tts_pad_embed || (trailing_len > 0 && !trailing_text)))
        return fail(c, QTTS_EINVAL, "predictor loop needs tts_pad_embed and trailing text");
    if (trailing_len < 0) return fail(c, QTTS_EINVAL, "trailing_len < 0");
    if (batch > 64) return fail(c, QTTS_ERANGE, "at most 64 streams per batch");
    const int B = batch, max_codes = params->max_codes;
    for (int b = 0; b < B; b++) n_frames[b] = 0;
    if (max_codes <= 0) return QTTS_OK;
    const Stack &ts = t->st;
    const int H = ts.hidden, V = t->vocab, cap = talker_kvs[0] ? talker_kvs[0]->cap : 0;
    for (int b = 0; b < B; b++) {
        qtts_kv *kv = talker_kvs[b];
        if (!kv) return fail(c, QTTS_EINVAL, "null talker cache");
        QTTS_TRY(check_kv(c, ts, kv));
        if (kv->cap != cap) return fail(c, QTTS_ESHAPE, "batched talker caches must share one capacity");
        if (kv->len + max_codes > kv->cap) return fail(c, QTTS_ERANGE, "talker cache too small");
        if (positions[b] < 0 || positions[b] + max_codes > t->max_pos)
            return fail(c, QTTS_ERANGE, "positions beyond the RoPE table");
    }
    if (!talker_only && p->talker_hidden != H) return fail(c, QTTS_ESHAPE, "predictor input width != talker hidden");
    // matrix-core operand copies
    if (t->mfma_state == 0) QTTS_TRY(make_talker_mfma(t));
    QTTS_TRY(make_head_mfma(t));
    if (t->mfma_state != 1 || t->head_mfma_state != 1)
        return fail(c, QTTS_ESHAPE, "batched loop: a talker weight cannot use the matrix cores");
    if (!talker_only) {
        if (p->mfma_state == 0) QTTS_TRY(make_predictor_mfma(p));
        QTTS_TRY(make_predictor_tables(p));
        if (p->mfma_state != 1) return fail(c, QTTS_ESHAPE, "batched loop: a predictor weight cannot use the matrix cores");
    }
    const Stack *ps = talker_only ? nullptr : &p->st;
    const int hp = ps ? ps->hidden : 0, pcap = talker_only ? 0 : p->groups + 1, G = talker_only ? 0 : p->groups;
    const int t_raw = std::max(ts.nq * ts.hd + 2 * ts.nkv * ts.hd, 2 * ts.inter);
    const int p_raw = ps ? std::max(ps->nq * ps->hd + 2 * ps->nkv * ps->hd, 2 * ps->inter) : 0;
    const int qd_max = std::max(ts.nq * ts.hd, ps ? ps->nq * ps->hd : 0);
    const size_t ncodes = (size_t)16 * max_codes;

    DevAllocs A;
    LoopState *S = nullptr;
    uint32_t *dcodes = nullptr;
    float *trail = nullptr, *pad = nullptr, *x = nullptr, *in2 = nullptr, *lg = nullptr, *raw = nullptr, *q = nullptr;
    float *att = nullptr, *xp = nullptr, *plog = nullptr, *pk = nullptr, *pv = nullptr;
    const float **tab = nullptr;
    int *pos2 = nullptr;
    QTTS_TRY(A.get(c, &S, (size_t)B));
    QTTS_TRY(A.get(c, &dcodes, (size_t)B * ncodes));
    QTTS_TRY(A.get(c, &trail, (size_t)B * std::max(trailing_len, 1) * H));
    QTTS_TRY(A.get(c, &pad, (size_t)H));
    QTTS_TRY(A.get(c, &x, (size_t)B * H));
    QTTS_TRY(A.get(c, &in2, (size_t)2 * B * H));
    QTTS_TRY(A.get(c, &lg, (size_t)B * V));
    QTTS_TRY(A.get(c, &raw, (size_t)2 * B * std::max(t_raw, p_raw)));
    QTTS_TRY(A.get(c, &q, (size_t)2 * B * qd_max));
    QTTS_TRY(A.get(c, &att, (size_t)2 * B * qd_max));
    QTTS_TRY(A.get(c, &tab, (size_t)8 * B));
    if (!talker_only) {
        QTTS_TRY(A.get(c, &xp, (size_t)2 * B * hp));
        QTTS_TRY(A.get(c, &plog, (size_t)B * p->vocab));
        const size_t pstride = (size_t)ps->layers * ps->nkv * pcap * ps->hd;
        QTTS_TRY(A.get(c, &pk, (size_t)B * pstride));
        QTTS_TRY(A.get(c, &pv, (size_t)B * pstride));
        QTTS_TRY(A.get(c, &pos2, (size_t)2 * B));
    }
    // row tables: talker caches [B]; predictor caches, two rows per stream
    // for the first pass [2B] and one per stream after it [B]
    std::vector<const float *> htab((size_t)8 * B, nullptr);
    std::vector<int> hpos2((size_t)2 * B);
    for (int b = 0; b < B; b++) {
        htab[b] = talker_kvs[b]->k;
        htab[B + b] = talker_kvs[b]->v;
        if (!talker_only) {
            const size_t pstride = (size_t)ps->layers * ps->nkv * pcap * ps->hd;
            const float *kb = pk + b * pstride, *vb = pv + b * pstride;
            htab[2 * B + 2 * b] = htab[2 * B + 2 * b + 1] = kb;  // [2B] K
            htab[4 * B + 2 * b] = htab[4 * B + 2 * b + 1] = vb;  // [2B] V
            htab[6 * B + b] = kb;                                // [B] K
            htab[7 * B + b] = vb;                                // [B] V
            hpos2[2 * b] = 0;
            hpos2[2 * b + 1] = 1;
        }
    }
    HIP_TRY(c, hipMemcpyAsync(tab, htab.data(), htab.size() * sizeof(float *), hipMemcpyHostToDevice, c->stream));
    if (!talker_only)
        HIP_TRY(c, hipMemcpyAsync(pos2, hpos2.data(), hpos2.size() * sizeof(int), hipMemcpyHostToDevice, c->stream));
    const float *const *t_k = tab, *const *t_v = tab + B;
    const float *const *p_k2 = tab + 2 * B, *const *p_v2 = tab + 4 * B;
    const float *const *p_k1 = tab + 6 * B, *const *p_v1 = tab + 7 * B;
    // initial state
    std::vector<LoopState> init((size_t)B);
    for (int b = 0; b < B; b++) {
        init[b] = LoopState{};
        init[b].pos = positions[b];
        init[b].kvlen = talker_kvs[b]->len;
        init[b].rng = seeds[b];
    }
    HIP_TRY(c, hipMemcpyAsync(S, init.data(), sizeof(LoopState) * B, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipMemsetAsync(dcodes, 0, (size_t)B * ncodes * sizeof(uint32_t), c->stream));
    if (trailing_len > 0)
        HIP_TRY(c, hipMemcpyAsync(trail, trailing_text, sizeof(float) * B * trailing_len * H, hipMemcpyHostToDevice,
                                  c->stream));
    if (tts_pad_embed)
        HIP_TRY(c, hipMemcpyAsync(pad, tts_pad_embed, sizeof(float) * H, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(c, hipMemcpyAsync(lg, logits, sizeof(float) * B * V, hipMemcpyHostToDevice, c->stream));
    if (!talker_only)
        HIP_TRY(c, hipMemcpy2DAsync(in2, sizeof(float) * 2 * H, last_hidden, sizeof(float) * H, sizeof(float) * H, B,
                                    hipMemcpyHostToDevice, c->stream));
    const long long SS = (long long)sizeof(LoopState), SW = SS / 4;
    const int tsplit = attn_nsplit(cap, 8);  // 8 splits measured ahead of 16 and 32 for 16 rows at 1064 positions
    RowTab TR;
    TR.k = t_k;
    TR.v = t_v;
    TR.pos = &S[0].pos;
    TR.kv = &S[0].kvlen;
    TR.stride = (int)SW;
    TR.cap = cap;

    // one frame for every stream; captured once into a HIP graph and
    // replayed (QTTS_NO_GRAPH=1: enqueued eagerly every frame)
    const float *ptab = !talker_only && p->tab_state == 1 ? p->tab : nullptr;  // the predictor's input table
    auto enqueue_frame_batch = [&]() -> qtts_status {
        // 1. code 0 of every stream (sample_token, src/generate_new.rs:329-391)
        SampleParams sp{};
        sp.logits = lg;
        sp.vocab = V;
        sp.temperature = params->sampler.temperature;
        sp.top_k = params->sampler.top_k;
        sp.penalty = params->sampler.repetition_penalty;
        sp.greedy = params->sampler.greedy;
        sp.prev = S[0].prev;
        sp.n_prev = 16;
        sp.rng = &S[0].rng;
        sp.token_out = &S[0].cur[0];
        sp.status = &S[0].status;
        sp.done = &S[0].done;
        sp.stop_on_eos = params->stop_on_eos;
        sp.eos = params->codec_eos_id;
        sp.codes = dcodes;
        sp.frame = &S[0].frame;
        sp.max_codes = max_codes;
        sp.prev_out = &S[0].prev[0];
        sp.batch = B;
        sp.state_stride = SS;
        sp.logits_stride = V;
        sp.codes_stride = (long long)ncodes;
        launch_sample(c->stream, sp);
        QTTS_TRY(check_launch(c, "k_sample"));
        // 2. the predictor's 15 passes (generate_acoustic_codes, src/code_predictor.rs:218-273)
        if (!talker_only) {
            launch_embed_rows(c->stream, t->emb, &S[0].cur[0], SW, B, in2 + H, 2LL * H);
            QTTS_TRY(check_launch(c, "k_embed_rows"));
            for (int g = 0; g < G; g++) {
                RowTab PR;
                PR.cap = pcap;
                int M;
                if (g == 0) {
                    M = 2 * B;
                    if (p->identity_proj)
                        HIP_TRY(c, hipMemcpyAsync(xp, in2, sizeof(float) * 2 * B * hp, hipMemcpyDeviceToDevice,
                                                  c->stream));
                    else
                        QTTS_TRY(run_gemm_mfma(c, p->mfma_in, in2, M, H, MFMA_ROWS_PLAIN, nullptr, xp, hp, p->bias,
                                               false));
                    PR.k = p_k2;
                    PR.v = p_v2;
                    PR.pos = pos2;
                    PR.kv = pos2;
                    PR.stride = 1;
                } else {
                    M = B;
                    if (!ptab) {  // with the table, the previous argmax filled xp
                        float *dst = p->identity_proj ? xp : in2;
                        launch_embed_rows(c->stream, p->emb[g - 1], &S[0].cur[g], SW, B, dst,
                                          p->identity_proj ? hp : H);
                        QTTS_TRY(check_launch(c, "k_embed_rows"));
                        if (!p->identity_proj)
                            QTTS_TRY(run_gemm_mfma(c, p->mfma_in, in2, M, H, MFMA_ROWS_PLAIN, nullptr, xp, hp,
                                                   p->bias, false));
                    }
                    PR.k = p_k1;
                    PR.v = p_v1;
                    PR.pos0 = g + 1;
                    PR.kv0 = g + 1;
                }
                QTTS_TRY(layers_batched(c, *ps, p->mfma.data(), PR, xp, M, raw, q, att, 1, g > 0));
                // head g on the last row of each stream
                const float *hx = g == 0 ? xp + hp : xp;
                const int hld = g == 0 ? 2 * hp : hp;
                QTTS_TRY(run_gemm_mfma(c, p->mfma_heads[(size_t)g], hx, B, hld, MFMA_ROWS_RMSNORM, ps->final_g, plog,
                                       p->vocab, nullptr, false));
                // with the table, the argmax also writes the next pass's
                // input rows: the projected embedding of each stream's code
                const float *nt = ptab && g + 1 < G ? ptab + (size_t)g * p->tab_rows * hp : nullptr;
                launch_argmax_rows(c->stream, plog, B, p->vocab, &S[0].cur[1 + g], SW, &S[0].status, SS, nt,
                                   p->tab_rows, hp, xp, hp);
                QTTS_TRY(check_launch(c, "k_argmax_rows"));
            }
        }
        // 3. the next talker input (src/generate_new.rs:270-286)
        EmbSumParams e{};
        e.mode = 0;  // talker-only: num_groups 0 gives codec_emb[code0] alone
        e.codec_emb = t->emb;
        if (!talker_only)
            for (int g = 0; g < G; g++) e.group_emb[g] = p->emb[g];
        e.num_groups = G;
        e.cur = S[0].cur;
        e.trailing = trail;
        e.trailing_len = trailing_len;
        e.pad = pad;
        e.frame = &S[0].frame;
        e.out = x;
        e.hidden = H;
        e.d_done = &S[0].done;
        e.codes = dcodes;
        e.max_codes = max_codes;
        e.prev = S[0].prev;
        e.batch = B;
        e.state_stride = SS;
        e.trailing_stride = (long long)trailing_len * H;
        e.out_stride = H;
        e.codes_stride = (long long)ncodes;
        launch_embed_sum(c->stream, e);
        QTTS_TRY(check_launch(c, "k_embed_sum"));
        // 4. talker step for every stream, then the codec head
        QTTS_TRY(layers_batched(c, ts, t->mfma.data(), TR, x, B, raw, q, att, tsplit, true));
        QTTS_TRY(run_gemm_mfma(c, t->head_mfma, x, B, H, MFMA_ROWS_RMSNORM, ts.final_g, lg, V, nullptr, false,
                               talker_only ? nullptr : in2, 2 * H));
        launch_advance(c->stream, S, 1, B);
        QTTS_TRY(check_launch(c, "k_advance"));
            return QTTS_OK;
    };
    // every GEMM's scratch, reserved before capture
    QTTS_TRY(mfma_reserve(c, H, ts.nq * ts.hd + 2 * ts.nkv * ts.hd, B));
    QTTS_TRY(mfma_reserve(c, ts.nq * ts.hd, H, B));
    QTTS_TRY(mfma_reserve(c, H, 2 * ts.inter, B));
    QTTS_TRY(mfma_reserve(c, ts.inter, H, B));
    QTTS_TRY(mfma_reserve(c, H, V, B));
    if (!talker_only) {
        if (!p->identity_proj) QTTS_TRY(mfma_reserve(c, H, hp, 2 * B));
        QTTS_TRY(mfma_reserve(c, hp, ps->nq * ps->hd + 2 * ps->nkv * ps->hd, 2 * B));
        QTTS_TRY(mfma_reserve(c, ps->nq * ps->hd, hp, 2 * B));
        QTTS_TRY(mfma_reserve(c, hp, 2 * ps->inter, 2 * B));
        QTTS_TRY(mfma_reserve(c, ps->inter, hp, 2 * B));
        QTTS_TRY(mfma_reserve(c, hp, p->vocab, B));
    }
    const bool use_graph = std::getenv("QTTS_NO_GRAPH") == nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    if (use_graph) {
        HIP_TRY(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        const qtts_status st = enqueue_frame_batch();
        hipError_t e = hipStreamEndCapture(c->stream, &graph);
        if (st != QTTS_OK || e != hipSuccess) {
            if (graph) (void)hipGraphDestroy(graph);
            return st != QTTS_OK ? st : fail(c, QTTS_EDEVICE, std::string("graph capture: ") + hipGetErrorString(e));
        }
        e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(graph);
            return fail(c, QTTS_EDEVICE, std::string("graph instantiate: ") + hipGetErrorString(e));
        }
    }
    qtts_status rc = QTTS_OK;
    for (int f = 0; f < max_codes && rc == QTTS_OK; f++) {
        if (use_graph) {
            const hipError_t e = hipGraphLaunch(exec, c->stream);
            if (e != hipSuccess) rc = fail(c, QTTS_EDEVICE, std::string("graph launch: ") + hipGetErrorString(e));
        } else {
            rc = enqueue_frame_batch();
        }
    }
    // No replay may still be in flight when the executable graph goes away.
    if (rc == QTTS_OK) rc = sync(c);
    else (void)hipStreamSynchronize(c->stream);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    QTTS_TRY(rc);
    std::vector<LoopState> fin((size_t)B);
    HIP_TRY(c, hipMemcpy(fin.data(), S, sizeof(LoopState) * B, hipMemcpyDeviceToHost));
    for (int b = 0; b < B; b++)
        if (fin[b].status != 0) return fail(c, (qtts_status)fin[b].status, "NaN logits during generation");
    HIP_TRY(c, hipMemcpy(codes, dcodes, (size_t)B * ncodes * sizeof(uint32_t), hipMemcpyDeviceToHost));
    for (int b = 0; b < B; b++) {
        n_frames[b] = fin[b].frame;
        talker_kvs[b]->len += fin[b].frame;
    }
    return QTTS_OK;
}

}  // extern "C"
