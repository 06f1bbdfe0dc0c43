// internal.h — device-side data layout and kernel parameter blocks shared by
// the HIP kernels (kernels.hip) and the host runtime (api.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace qtts {

// Repacked Q4 weight ("panel-major").  The reference stores packed[k][n/2]
// and scales[k][n/32] (src/gemv.rs:26-31).  On the device the 32 output
// columns of one scale group form a panel; panel p holds, for every input row
// k, the 16 packed bytes of columns [32p, 32p+32) (same nibble order as the
// reference) followed in a separate array by that row's binary16 scale:
//   wq[p*K + k] = packed[k][16p .. 16p+16)     (one 128-bit load)
//   ws[p*K + k] = scales[k][p]
// A wavefront reading 64 consecutive rows of one panel reads 1 KiB of
// contiguous weights and 128 B of contiguous scales.  Total bytes are exactly
// the reference's Weight::memory_bytes().
struct DevQ4 {
    const uint4 *wq;
    const uint16_t *ws;
    int K;  // input rows
    int N;  // output columns (multiple of 32); panels = N / 32
};

// The same weight in the MFMA B-operand order (csrc/mfma.hip), made on
// first use by a GEMM of >= 8 rows:
//   wm[(p * K/16 + s) * 64 + l]: panel p, 16-row step s, lane l: column
//     32p + l%32, rows 16s + 8(l/32) + i (i < 8), nibble i at bits
//     4*(i/2) + 16*(i%2) -- rows 2j and 2j+1 are the two halves of
//     (word >> 4j) & 0x000F000F;
//   sa[p*K + k], sb[p*K + k]: the row's binary16 scale split exactly into
//     its top 7 and low 4 significand bits (s = sa + sb).
struct DevQ4Mfma {
    const uint32_t *wm;
    const uint16_t *sa, *sb;
    int K, N;
};

// Row prologues of the MFMA GEMM's input split.
enum MfmaRowsMode { MFMA_ROWS_PLAIN = 0, MFMA_ROWS_RMSNORM = 1, MFMA_ROWS_SWIGLU = 2 };
constexpr int kMfmaRowsMaxK = 8192;

struct MfmaRowsParams {
    const float *x;  // row m at x + m * ldx (SWIGLU: gate [0, K), up [K, 2K))
    int ldx, K, M, Mpad, mode;
    const uint16_t *gamma;  // RMSNORM weight (binary16 bits)
    _Float16 *xh, *xl;      // [Mpad / 32][K / 16][64][8], the MFMA A-operand order
    int *rexp;              // [Mpad] row exponents
    float *norm_out;        // optional: the prologue's rows (f32) at norm_out[m * ldn + k]
    int ldn;
};

// apply_qk_norm + RoPE + KV append over M rows of a fused QKV projection
// (the EPI_QKV epilogue of the GEMV, as a kernel of its own).
struct QkvRowsParams {
    const float *raw;  // row m at raw + m * ldr: [q heads | k heads | v heads] x head_dim
    int ldr, M;
    int n_q_heads, n_kv_heads, head_dim;
    const uint16_t *q_norm, *k_norm;
    const float *rope_cos, *rope_sin;
    int rope_rows, rope_skip_oob;
    float *q;  // [M][n_q_heads * head_dim], ldq
    int ldq;
    float *kcache, *vcache;  // [n_kv_heads][kv_cap][head_dim]
    int kv_cap;
    int pos0, row0;  // RoPE position and cache row of row 0
    // independent rows (batched streams): with row_k set, row m's layer-0
    // K/V bases are row_k[m] / row_v[m] (this layer at + layer_off), its
    // position pos0 + row_pos[m * row_stride] and cache row
    // row0 + row_kv[m * row_stride] (a null table counts as zeros)
    const float *const *row_k, *const *row_v;
    const int *row_pos, *row_kv;
    int row_stride;
    long long layer_off;
};

// ---- speech decoder (csrc/decoder.hip) ----
constexpr int kDecMaxWindow = 512;   // sliding window of the decoder attention
constexpr int kDecMaxHeadDim = 256;
constexpr int kDecMaxSlots = 64;  // slots of one tensor's max |x| (SnakeBeta -> k_dec_conv_mfma)
constexpr int kConvStage = 2;     // 16-row K steps per LDS stage of k_dec_conv_mfma (ksteps is a multiple)

struct DecGatherParams {
    const uint32_t *codes;  // [groups][ld]
    int ld, cd, cb_size, num_rest;
    const float *first;          // [cb_size][cd]
    const float *const *rest;    // device array of num_rest codebook pointers
    float *e0, *es;              // [T][cd]
    int *status;                 // set to 1 for a code >= cb_size
};

enum DecAct { DEC_ACT_NONE = 0, DEC_ACT_GELU = 1 };
enum DecEpi { DEC_EPI_STORE = 0, DEC_EPI_ACCUM = 1, DEC_EPI_SCALED_RESID = 2, DEC_EPI_RESID_IN = 3, DEC_EPI_CLAMP = 4 };

// A convolution or linear layer on the matrix cores (k_dec_conv_mfma) as a
// causal convolution: output (m, n) = act(sum_{tap, ci} A(m, ci, tap) *
// x(ci, n + (tap - (ksize - 1)) * dilation) + bias[m]) (x zero before n = 0),
// combined into c by `epi` (STORE: =, ACCUM: +=, SCALED_RESID: += scale[m] *,
// RESID_IN: = resid + scale[m] *, CLAMP: = clamp to [-1, 1]).  A: weights pre-split into
// binary16 hi + lo in the MFMA A-operand order, one 16-row K step per
// (16-channel block, tap) with the taps inner (the channels padded to a
// multiple of 16 with zero weights); x(ci, p) = x[ci * sxc + p * sxn],
// split on the fly.  A linear
// layer is the case ksize = 1 with m the output feature and n the row.
constexpr int kDecMaxPhases = 8;  // output phases of one transposed-convolution launch

struct DecConvMfmaParams {
    const _Float16 *wh, *wl;  // [mtiles][ksteps][64][8]; row m = 32 * tile + lane % 32
    int ew;                   // the weights were scaled by 2^ew
    int M, mtiles, ksteps;    // output channels, 32-row tiles, 16-row K steps (ksize * cin16 / 16,
                              // rounded up to a multiple of kConvStage with zero weights)
    int cin, cin16, ksize, dilation, len;  // len: output positions n
    const float *x;
    long long sxc, sxn;       // x strides of a channel and a position
    const unsigned *xmax;     // [kDecMaxSlots]: bits of max |x| over the slots
    const float *bias;        // [M] or null
    const float *scale;       // [M]: DEC_EPI_SCALED_RESID / DEC_EPI_RESID_IN (null: 1)
    int act, epi;             // DecAct, DecEpi
    float *c;                 // output (m, n) at c[m * ldc + n * out_stride + phase]
    long long ldc;
    long long out_stride;
    int phase;
    const float *resid;       // DEC_EPI_RESID_IN: at the output's index (may be c)
    // nphase > 1: one launch runs the output phases 0 .. nphase-1 of a
    // transposed convolution (grid z = phase); phase p's weights are
    // ph_wh[p] / ph_wl[p] (wh, wl and phase are then unused)
    int nphase;
    const _Float16 *ph_wh[kDecMaxPhases], *ph_wl[kDecMaxPhases];
};

struct DecAttnParams {
    const float *q, *k, *v;  // rows of heads * hd values, ld apart (0: heads * hd)
    int ld;
    float *out;
    int T, heads, hd, window;
    float scale;
};

struct GemmMfmaParams {
    DevQ4Mfma w;
    const _Float16 *xh, *xl;  // the scaled rows split into binary16 hi + lo (MfmaRowsParams order)
    const int *rexp;          // [32 * MT]: row m was scaled by 2^rexp[m]
    int M;                    // rows of this pass (<= 32 * MT)
    float *part;              // [kc][32 * MT][N] when kc > 1
    unsigned *counters;       // [N / 32], zero between launches
    const float *bias;        // optional
    float *y;                 // y[m * ldy + n] (+)= result
    int ldy, accumulate;
};

constexpr int kGemvThreads = 256;
constexpr int kGemvWideThreads = 1024;  // the one-row GEMV's block for 2048 < K <= 8192
constexpr int kMaxM = 4;          // rows per GEMV launch (prefill chunks)
constexpr int kMfmaMinRows = 8;   // GEMMs of at least this many rows run on the matrix cores
constexpr int kMaxGroups = 15;    // predictor code groups
constexpr int kAttnThreads = 256;
constexpr int kAttnMaxChunk = 256;  // positions per attention split block
constexpr int kMaxHeadDim = 128;
constexpr int kSampleThreads = 1024;

enum Prologue : int {
    PRO_PLAIN = 0,    // x[m][k] = x[m*ldx + k]
    PRO_RMSNORM = 1,  // x[m][k] = rms_norm_f16(src row m, gamma)[k]
    PRO_EMBED = 2,    // x[0][k] = embed_lookup(emb, *emb_token)[k]
};

enum Epilogue : int {
    EPI_STORE = 0,   // y[m*ldy + j] = gemv (+ bias[j])
    EPI_RESID = 1,   // y[m*ldy + j] += gemv
    EPI_SWIGLU = 2,  // y[m*ldy + j] = silu(gate_j) * up_j; gate = cols [0,N/2), up = [N/2,N)
    EPI_QKV = 3,     // per head: QK-norm + RoPE, q -> y, k/v -> KV cache
};

enum Final : int {
    FIN_NONE = 0,
    FIN_ARGMAX = 1,  // after all groups: argmax of y[0..N) -> *argmax_out
};

struct GemvParams {
    DevQ4 w;
    int M;
    int kc;   // K chunks (blocks per panel)
    int rpt;  // rows per thread per chunk; chunk = 256*rpt rows
    int prologue, epilogue, fin;
    // input
    const float *x;
    int ldx;
    const uint16_t *gamma;  // PRO_RMSNORM
    int norm_src_row0;      // PRO_RMSNORM: source row of output row 0 (m -> row0 + m)
    float *norm_out;        // PRO_RMSNORM: optional, receives the normed rows
    int ldn;
    DevQ4 emb;                   // PRO_EMBED
    const uint32_t *emb_token;   // PRO_EMBED: device token index
    // output
    float *y;
    int ldy;
    const float *bias;
    // EPI_QKV
    int n_q_heads, n_kv_heads, head_dim;
    const uint16_t *q_norm, *k_norm;
    const float *rope_cos, *rope_sin;
    int rope_rows;
    int rope_skip_oob;
    float *kcache, *vcache;  // this layer: [kv_heads][cap][head_dim]
    int kv_cap;
    const int *d_pos;  // rope position of row m = (*d_pos or pos_const) + m
    int pos_const;
    const int *d_kvlen;  // cache row of row m = (*d_kvlen or kvlen_const) + m
    int kvlen_const;
    // FIN_ARGMAX
    uint32_t *argmax_out;
    int *status;  // set to QTTS_ENAN on NaN
    // scratch
    float *partial;      // [kc][M][N]
    unsigned *counters;  // [groups + 1], zero between launches
    const int *d_done;   // skip the launch when *d_done != 0
};

struct AttnParams {
    const float *q;  // [M][nq*hd]
    int ldq;
    const float *kcache, *vcache;  // this layer: [nkv][cap][hd]
    int kv_cap;
    int nq, nkv, hd;
    const int *d_kvlen;  // cache length before this step's rows were appended
    int kvlen_const;
    int nsplit;
    float scale;
    float *part;         // [M][nq][nsplit][hd + 2]
    unsigned *counters;  // [M][nkv]
    float *out;          // [M][nq*hd]
    int ldo;
    const int *d_done;
    // independent rows (batched streams): with row_k set, row m attends to
    // its own cache (row_k[m] / row_v[m] + layer_off) over
    // kvlen_const + row_kv[m * row_stride] + 1 positions
    const float *const *row_k, *const *row_v;
    const int *row_kv;
    int row_stride;
    long long layer_off;
    // one new row per stream (batched decode): with raw set, q is not read;
    // every block QK-norms and rotates its kv head's query heads from the
    // raw GEMM output (row m at raw + m * ldr, [q | k | v] heads x hd), and
    // the block whose split holds the new position (kvlen_const +
    // row_kv[m * row_stride]) does the same for k, appends k and v to the
    // cache there and uses them from LDS -- the work of k_qkv_rows
    const float *raw;
    int ldr;
    const uint16_t *q_norm, *k_norm;
    const float *rope_cos, *rope_sin;
    int rope_rows, rope_skip_oob;
    const int *row_pos;  // RoPE position pos0 + row_pos[m * row_stride]
    int pos0;
};

// Device-resident state of one generation loop (one per talker).
struct LoopState {
    int pos;           // talker RoPE position
    int kvlen;         // talker cache length
    int frame;         // frames produced
    int done;          // EOS seen (stop_on_eos) or error
    int status;        // qtts_status of the device side
    int pad0;
    uint64_t rng;      // simple_rand state
    uint32_t prev[16]; // prev_tokens
    uint32_t cur[16];  // codes of the current frame
};

struct SampleParams {
    const float *logits;
    int vocab;
    float temperature;
    int top_k;
    float penalty;
    int greedy;
    const uint32_t *prev;
    int n_prev;
    uint64_t *rng;
    uint32_t *token_out;
    int *status;
    // loop integration (all optional)
    int *done;
    int stop_on_eos;
    uint32_t eos;
    uint32_t *codes;  // codes[frame] of group 0
    const int *frame;
    int max_codes;
    uint32_t *prev_out;  // prev_tokens[0] = token
    // batched streams: block b works on stream b; every pointer above into a
    // LoopState moves by b * state_stride bytes, logits by b * logits_stride
    // floats, codes by b * codes_stride words
    int batch;
    long long state_stride, logits_stride, codes_stride;
};

struct EmbSumParams {
    int mode;                     // 0: full next-step input, 1: acoustic sum only
    DevQ4 codec_emb;              // talker codec_embedding
    DevQ4 group_emb[kMaxGroups];  // predictor codec_embeddings
    int num_groups;
    const uint32_t *cur;  // cur[0] = code0, cur[1+g] = acoustic code g
    const float *trailing;
    int trailing_len;
    const float *pad;
    const int *frame;
    float *out;       // combined embedding
    int hidden;
    const int *d_done;
    // frame bookkeeping: codes[g][frame] = cur[g], prev[g] = cur[g] for g >= 1
    uint32_t *codes;
    int max_codes;
    uint32_t *prev;
    // batched streams (grid.y = batch): LoopState pointers (cur, frame,
    // d_done, prev) move by y * state_stride bytes, trailing by
    // y * trailing_stride floats, out by y * out_stride floats, codes by
    // y * codes_stride words
    int batch;
    long long state_stride, trailing_stride, out_stride, codes_stride;
};

// Launchers (kernels.hip).
void launch_gemv(hipStream_t st, const GemvParams &p);
void launch_attention(hipStream_t st, const AttnParams &p, int M);
void launch_sample(hipStream_t st, const SampleParams &p);
void launch_embed_row(hipStream_t st, const DevQ4 &w, const uint32_t *d_token, float *out, const int *d_done);
void launch_repack_mfma(hipStream_t st, const DevQ4 &w, uint32_t *wm, uint16_t *sa, uint16_t *sb, int *too_large);
void launch_mfma_rows(hipStream_t st, const MfmaRowsParams &p);
void launch_qkv_rows(hipStream_t st, const QkvRowsParams &p);
void launch_dec_gather(hipStream_t st, const DecGatherParams &p, int frames);
void launch_dec_rmsnorm(hipStream_t st, const float *x, const float *gamma, int rows, int n, float eps, float *out);
void launch_dec_rope(hipStream_t st, float *q, float *k, int T, int heads, int hd, const float *cs, const float *sn,
                     int rows, int ld);  // q, k rows ld apart
void launch_dec_attn(hipStream_t st, const DecAttnParams &p);
// out[t][j] = silu(g[t * ld + j]) * u[t * ld + j] for rows t < rows, j < width (out rows width apart)
void launch_dec_swiglu(hipStream_t st, const float *g, const float *u, int rows, int width, int ld, float *out);
void launch_dec_dwconv(hipStream_t st, const float *x, const float *w, const float *b, int ch, int len, int ks,
                       float *out);
void launch_dec_lnorm(hipStream_t st, const float *x, const float *g, const float *b, int ch, int len, float eps,
                      float *out);
void launch_dec_snake(hipStream_t st, const float *x, const float *alpha, const float *beta, int ch, int len,
                      float *out, unsigned *amax = nullptr, const float *add = nullptr, float *sum = nullptr);
void launch_dec_fill_u32(hipStream_t st, unsigned *p, int n, unsigned v);
void launch_dec_absmax(hipStream_t st, const float *x, size_t n, unsigned *amax);
void launch_dec_conv_repack(hipStream_t st, const float *w, long long sm, long long sci, int k0, int kd, int M, int cin,
                            int taps, int cin16, int mtiles, int ksteps, int ew, _Float16 *wh, _Float16 *wl);
void launch_dec_conv_mfma(hipStream_t st, const DecConvMfmaParams &p);
void launch_gemm_mfma(hipStream_t st, const GemmMfmaParams &p, int mt, int sw, int kc);
void launch_embed_sum(hipStream_t st, const EmbSumParams &p);
void launch_advance(hipStream_t st, LoopState *s, int frame_step, int batch = 1);
// Prompt rows of prefill_custom_voice: out[r] = a[r] (+ b[r] when b[r] is
// set), H floats per row, r < L <= 10.
struct PromptRowsParams {
    const float *a[10];
    const float *b[10];
    int L, H;
    float *out;
};
void launch_prompt_rows(hipStream_t st, const PromptRowsParams &p);
// x[i] = silu(x[i]) = x / (1 + exp(-x)) for i < n (src/gemv.rs:447-451).
void launch_silu(hipStream_t st, float *x, long long n);
// generate::sample_top_k (src/generate.rs:50-84) on one workgroup, vocab <= 4096.
struct TopKParams {
    const float *logits;
    int vocab;
    float temperature;
    int top_k;
    uint64_t *rng;
    uint32_t *token_out;
    int *status;
};
constexpr int kTopKMaxVocab = 4096;
void launch_sample_top_k(hipStream_t st, const TopKParams &p);
void launch_embed_rows(hipStream_t st, const DevQ4 &w, const uint32_t *tok, long long tok_stride, int rows, float *out,
                       long long out_stride);
// prefill_talker's rows: out[r] = text[slot[r]] if slot[r] >= 0, else the
// codec embedding of tok[r] (rows x H, H == w.N).
void launch_token_rows(hipStream_t st, const DevQ4 &w, const uint32_t *tok, const int *slot, const float *text,
                       int rows, float *out, int H);
void launch_argmax_rows(hipStream_t st, const float *logits, int rows, int n, uint32_t *out, long long out_stride,
                        int *status, long long status_stride, const float *table = nullptr, int table_rows = 0,
                        int width = 0, float *rows_out = nullptr, long long rows_ld = 0);
void launch_repack_q4(hipStream_t st, const uint8_t *packed, const uint16_t *scales, int K, int N, int col0,
                      int Ntot, uint4 *wq, uint16_t *ws);

// GEMV launch plan for a [K -> N] weight at M rows.
void plan_gemv(int K, int N, int M, int *kc, int *rpt);

// Limits of the allocation-free GEMV (qtts_gemv_device_static), whose split-K
// partials [chunks][rows][N] and arrival counters [N/32 + 1] live in a
// module-scope device array (kernels.hip), one per device.
constexpr int kStaticMaxK = 8192;  // <= 4 chunks of 2048 rows
constexpr int kStaticMaxN = 16384;
constexpr int kStaticMaxChunks = 4;
constexpr size_t kStaticPartialFloats = (size_t)kStaticMaxChunks * kMaxM * kStaticMaxN;
constexpr size_t kStaticCounterWords = kStaticMaxN / 32 + 64;
// Looks up (once per device, with that device current) and zeroes the
// device's copy of that array.
hipError_t static_scratch_setup(int device);
// Its device address for `device`, or null before setup.
void *static_scratch(int device);

}  // namespace qtts
