// engine.h — the persistent dataflow kernel that runs one frame of the
// per-code loop (or one talker step, or one predictor frame) in a single
// cooperative launch.
//
// A program is a list of ops (GEMV, attention, combine, argmax, sampler,
// embedding sum), each split into tasks.  Every block walks the ops in order
// and takes the tasks t with (t + rotation) % gridDim == blockIdx.  Values
// that cross blocks are "tagged": a 64-bit word holding the float bits and a
// 32-bit tag naming the op instance that wrote it.  A consumer spins on the
// words it needs until their tags match, so a dependency costs one device
// store + one device load (no grid barrier), and a block that has no task in
// an op moves on and issues the next op's weight loads while it waits.
//
// Deadlock freedom: tasks only wait on values of earlier ops, or (split-K
// owners) on the non-owner chunks of the same op, which come first in task
// order.  Every spin is bounded and also polls a shared abort word, so an
// error or EOS drains the grid.
#pragma once

#include "internal.h"

namespace qtts {

using tv_t = uint64_t;  // float bits | tag << 32

// One 512-thread block per CU: two waves per SIMD, so a task's
// accumulation is spread over twice the lanes and every wave has a partner
// to issue while it waits.  The kernel must then fit 256 registers a wave
// (VGPRs and AGPRs together).
constexpr int kEngThreads = 512;
constexpr int kEngWaves = kEngThreads / 64;
// Rows per thread of a GEMV task over a slice of `cols` columns of `np`
// panels (the K chunk is at most kEngThreads times this): a task's weights
// stay in registers from issue to use, cols / 8 dwords per row (one for 4
// columns).
constexpr int eng_rows_per_thread(int cols, int np) { return np == 2 || cols >= 16 ? 4 : cols == 4 ? 8 : 12; }
constexpr int kEngNormRows = 4;  // an RMSNorm input row has <= kEngThreads * 4 values
constexpr int kEngMaxM = 2;    // rows per GEMV (the predictor's 2-token prefill)
constexpr uint32_t kTagStride = 8192;  // tags reserved per code
constexpr int kEngCodesPerLaunch = 16;  // codes of the frame loop per cooperative launch
constexpr int kEngMaxSplit = 128;  // talker attention splits (<= 256 positions each: 32,768 cache rows)
constexpr int kEngSmemFloats = 10240;
constexpr int kEngLdsKvPos = 32;  // positions of an LDS-resident K/V cache (one kv head)
constexpr int kEngArgtabMax = 2048;  // logits of an EIN_ARGTAB input

enum EngOpKind : int { EOP_GEMV = 1, EOP_ATTN = 2, EOP_COMBINE = 3, EOP_ARGMAX = 4, EOP_SAMPLE = 5, EOP_EMBSUM = 6 };
enum EngIn : int { EIN_TV = 0, EIN_PLAIN = 1, EIN_EMBED = 2, EIN_ARGTAB = 3 };
enum EngEpi : int { EEPI_STORE = 0, EEPI_RESID = 1, EEPI_SWIGLU = 2 };

struct EngInput {
    int kind;
    int tag;              // EIN_TV: tag of tv; EIN_EMBED: tag of tok_tv
    const tv_t *tv;       // EIN_TV: the row (K values)
    const float *plain;   // EIN_PLAIN: the row, written by an earlier launch or the host
    DevQ4 emb;            // EIN_EMBED: x = emb row at the token
    const tv_t *tok_tv;   // EIN_EMBED: the token (integer in the value bits)
    const float *table;   // EIN_ARGTAB: x = table row at argmax(tv[0..n)) (a row of K floats;
    int table_rows;       //   a code past the last row gives zeros)
    int n;                // EIN_ARGTAB: logits in tv (<= kEngArgtabMax)
    int parts;            // EIN_TV with norm: 2 = the row is tv[k] + tv[K + k] (a split_out GEMV's
                          //   two chunks; K <= kEngThreads / 2 * kEngNormRows)
};

struct EngGemv {
    DevQ4 w;
    int M;       // rows (1 or 2): each row's tasks run separately (M x the one-row tasks)
    int kc;      // K chunks; chunk 0 owns the epilogue
    int kchunk;  // rows per chunk (multiple of kEngThreads, <= kEngThreads * eng_rows_per_thread(cols, panels))
    int cols;    // output columns per task: 32, 16, 8 or 4 (a slice of a 32-column panel);
                 // 32 or 16 for SwiGLU
    int epi;
    int norm;    // RMSNorm the input rows (rms_norm_f16)
    const uint16_t *gamma;
    EngInput in[kEngMaxM];
    const float *bias;
    const tv_t *resid;  // EEPI_RESID: y = resid + gemv
    int resid_tag, ld_resid;
    const float *resid_table;  // EEPI_RESID, M == 1: the residual is resid_table[code][col] instead,
    const tv_t *resid_code;    //   code a tagged integer (tag resid_tag), row stride ld_resid
    int resid_table_rows;
    int resid_parts;           // 2: the residual is resid[col] + resid[N + col]
    int split_out;             // kc == 2, NP == 1: chunk 1 publishes its sums as the output's second
                               //   part (out[m * ld_out + N + col]) and chunk 0 adds the residual and
                               //   bias to its own: no split-K wait; the consumers add the parts
    tv_t *out;
    int out_tag, ld_out;
    float *out_plain;  // optional plain copy of the output (read by a later launch)
    int ld_plain;
    float *norm_plain;  // optional: the normed input row M-1 (kc must be 1)
    tv_t *part;         // split-K partials [kc-1][M][N]
    int part_tag;
};

struct EngAttn {
    const tv_t *qkv;  // [M][ld_qkv]: q (nq*hd) | k (nkv*hd) | v (nkv*hd), before QK-norm/RoPE
    int qkv_tag, ld_qkv;
    int M, nq, nkv, hd;
    const uint16_t *q_norm, *k_norm;
    const float *rope_cos, *rope_sin;
    int rope_rows, rope_skip_oob;
    float *kcache, *vcache;  // this layer [nkv][cap][hd]
    int kv_cap;
    int from_state;          // position / cache length from the frame state (talker)
    int pos_const, len_const;
    int nsplit;
    int lds_kv;              // cached rows of this launch live in the block's LDS: every step
                             // of this layer runs task h on the same block (the host pins the
                             // rotation), which keeps kv head h's rows [0, len) there
    float scale;
    // lds_kv, M == 1: the raw q/k/v row is qkv_table[argmax(logits[0..logits_n))] (ld_qkv
    // floats; a code past the last row gives zeros) instead of the tagged qkv
    const float *qkv_table;
    int qkv_table_rows;
    const tv_t *logits;
    int logits_tag, logits_n;
    tv_t *part;  // nsplit > 1: [M][nq][nsplit][hd + 2]
    int part_tag;
    tv_t *out;   // nsplit == 1: [M][nq*hd]
    int out_tag;
};

struct EngCombine {
    const tv_t *part;
    int part_tag;
    int M, nq, hd, nsplit;
    tv_t *out;
    int out_tag;
};

struct EngArgmax {
    const tv_t *logits;
    int logits_tag, n;
    tv_t *code;  // one tagged integer
    int code_tag;
    int group;   // codes row this code is filed under
};

struct EngSample {
    const float *logits;  // plain, from the previous launch (or the host)
    int vocab;
    float temperature;
    int top_k;
    float penalty;
    int greedy;
    int stop_on_eos;
    uint32_t eos;
    int num_prev;  // prev_tokens entries (16)
    tv_t *tok;
    int tok_tag;
};

struct EngEmbSum {
    int mode;  // 0: codec_emb[tok] + sum_g group_emb[g][code_g] + text; 1: codec_emb[tok] only;
               // 2: copy the plain row `pad` (a host input)
    DevQ4 codec_emb;
    DevQ4 group_emb[kMaxGroups];
    const tv_t *code[kMaxGroups];
    int code_tag[kMaxGroups];
    int num_groups;
    const tv_t *tok;
    int tok_tag;
    const float *trailing;
    int trailing_len;
    const float *pad;
    int hidden;
    tv_t *out;
    int out_tag;
};

struct EngOp {
    int kind;
    int ntasks;
    int rot;  // task rotation across blocks
    int pad;
    union {
        EngGemv gemv;
        EngAttn attn;
        EngCombine comb;
        EngArgmax amax;
        EngSample samp;
        EngEmbSum emb;
    };
};

// Frame state, double-buffered across launches: a launch reads one copy and
// its sampler writes the other.
struct EngState {
    int pos;    // talker RoPE position
    int kvlen;  // talker cache length
    int frame;  // frames produced
    int pad;
    uint64_t rng;
};

struct EngArgs {
    const EngOp *ops;
    int nops;
    uint32_t tag_base;
    EngState *st;  // the two state copies: code f of the launch reads st[(st0 + f) & 1], its sampler
    int st0;       //   writes the other one
    int ncodes;    // codes (frames) run by this launch, one after another
    tv_t *bar;     // [grid + 1]: arrival words of the barrier between codes, then its release word
    int *done;    // abort word: EOS, error or timeout
    int *status;  // qtts_status of the device side
    uint32_t *codes;  // [16][max_codes]
    int max_codes;
    uint64_t *trace;  // optional [nops][grid][kTraceSlots]: wall clock at 0 start, 1 end, 2..7 inside a task;
                      // shader clock at 8 start, 9 end
};

constexpr int kTraceSlots = 10;

// cooperative: hipLaunchCooperativeKernel (the default, which guarantees
// that the whole grid is resident); otherwise an ordinary launch of the same
// grid (QTTS_ENGINE_LAUNCH=plain, for profiler runs: a process that made a
// cooperative launch holds the runtime's cooperative queue until exit).
hipError_t launch_engine(hipStream_t st, const EngArgs &a, int grid, bool cooperative);
int engine_max_grid();

}  // namespace qtts
