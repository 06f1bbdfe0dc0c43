// engine.hip — persistent dataflow kernel for the per-code loop (see engine.h).
#include <hip/hip_runtime.h>

#include <cmath>

#include "../../include/qtts.h"
#include "device_common.h"
#include "engine.h"

namespace qtts {

namespace {

constexpr uint32_t kSpinLimit = 1u << 23;

// Per-thread wait bookkeeping.  A thread that sees the abort word, or spins
// past the limit, marks itself bad and keeps executing the task with zeros
// (so every block barrier is still reached); the block leaves at the end of
// the task.
// TR: the traced kernel (QTTS_ENGINE_TRACE); the production kernel has no
// stamps, branches or trace pointer in its ops (they cost it ~4 %).
template <bool TR>
struct Ctl {
    static constexpr bool kTrace = TR;
    int *done;
    int *status;
    uint32_t spins;
    bool bad;
    uint64_t *tr;  // trace slots of this (op, block), or null (TR only)
};

// Trace stamp k (2..7) of the current task, thread 0 only.
template <class CT>
__device__ __forceinline__ void stamp(const CT &c, int k) {
    if constexpr (CT::kTrace)
        if (c.tr && threadIdx.x == 0) glb(c.tr)[k] = wall_clock64();
}

template <class CT>
__device__ __forceinline__ void fail_dev(CT &c, int code) {
    st_dev_i32(c.status, code);
    st_dev_i32(c.done, 1);
    c.bad = true;
}

template <class CT>
__device__ __forceinline__ bool must_stop(CT &c) {
    if (c.bad) return true;
    if ((++c.spins & 127u) == 0u) {
        if (ld_dev_i32(c.done)) {
            c.bad = true;
            return true;
        }
        if (c.spins > kSpinLimit) {
            fail_dev(c, QTTS_EDEVICE);
            return true;
        }
    }
    return false;
}

template <class CT>
__device__ __forceinline__ float wait_tv(const tv_t *p, uint32_t tag, CT &c) {
    uint64_t v = ld_dev_u64(p);
    while ((uint32_t)(v >> 32) != tag) {
        if (must_stop(c)) return 0.0f;
        __builtin_amdgcn_s_sleep(1);
        v = ld_dev_u64(p);
    }
    return __uint_as_float((uint32_t)v);
}

// Waits for `count` (<= N) words base[i*stride]: all loads are issued
// before any tag is checked, then only the stale ones are re-read.
template <int N, class CT>
__device__ __forceinline__ void wait_strided(const tv_t *base, size_t stride, int count, uint32_t tag, float (&out)[N],
                                             CT &c) {
    uint64_t v[N];
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = i < count ? ld_dev_u64(base + i * stride) : ((uint64_t)tag << 32);
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; i++) ok &= ((uint32_t)(v[i] >> 32) == tag);
        if (ok || must_stop(c)) break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < N; i++) v[i] = i < count ? ld_dev_u64(base + i * stride) : v[i];
    }
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __uint_as_float((uint32_t)v[i]);
}

// out[i] = a[i*stride] + b[i*stride] for i < count (<= N), one tag: all 2N
// loads are issued before any tag is checked.
template <int N, class CT>
__device__ __forceinline__ void wait_pair(const tv_t *a, const tv_t *b, size_t stride, int count, uint32_t tag,
                                          float (&out)[N], CT &c) {
    uint64_t va[N], vb[N];
#pragma unroll
    for (int i = 0; i < N; i++) {
        va[i] = i < count ? ld_dev_u64(a + i * stride) : ((uint64_t)tag << 32);
        vb[i] = i < count ? ld_dev_u64(b + i * stride) : ((uint64_t)tag << 32);
    }
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; i++) ok &= ((uint32_t)(va[i] >> 32) == tag) & ((uint32_t)(vb[i] >> 32) == tag);
        if (ok || must_stop(c)) break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < N; i++) {
            va[i] = i < count ? ld_dev_u64(a + i * stride) : va[i];
            vb[i] = i < count ? ld_dev_u64(b + i * stride) : vb[i];
        }
    }
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __uint_as_float((uint32_t)va[i]) + __uint_as_float((uint32_t)vb[i]);
}

// Same for a list of words with their own tags.
template <int N, class CT>
__device__ __forceinline__ void wait_list(const tv_t *const (&p)[N], const uint32_t (&tag)[N], int count,
                                          float (&out)[N], CT &c) {
    uint64_t v[N];
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = i < count ? ld_dev_u64(p[i]) : ((uint64_t)tag[i] << 32);
    for (;;) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; i++) ok &= ((uint32_t)(v[i] >> 32) == tag[i]);
        if (ok || must_stop(c)) break;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < N; i++) v[i] = i < count ? ld_dev_u64(p[i]) : v[i];
    }
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __uint_as_float((uint32_t)v[i]);
}

template <class CT>
__device__ __forceinline__ uint32_t wait_tv_u32(const tv_t *p, uint32_t tag, CT &c) {
    return __float_as_uint(wait_tv(p, tag, c));
}

__device__ __forceinline__ void put_tv(tv_t *p, float x, uint32_t tag) {
    st_dev_u64(p, ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(x));
}

__device__ __forceinline__ void put_tv_u32(tv_t *p, uint32_t x, uint32_t tag) {
    st_dev_u64(p, ((uint64_t)tag << 32) | (uint64_t)x);
}

// Sum of the block's kEngWaves per-wave values v[w * stride], as a pairwise
// tree (fixed order: the result does not depend on timing).
__device__ __forceinline__ float waves_sum(const float *v, int stride) {
    float t[kEngWaves];
#pragma unroll
    for (int w = 0; w < kEngWaves; w++) t[w] = v[w * stride];
#pragma unroll
    for (int h = kEngWaves / 2; h >= 1; h /= 2)
#pragma unroll
        for (int w = 0; w < h; w++) t[w] = t[w] + t[w + h];
    return t[0];
}

// sample_argmax (src/code_predictor.rs:328-334) of n <= kEngThreads * NA
// tagged logits over the block: the last index of the maximum (-1 when every
// value is NaN).  Every thread gets the result; *anynan says whether any
// logit was NaN.  scr: 2 * kEngWaves words of LDS that no thread touches
// again before the next block barrier.
template <int NA, class CT>
__device__ __forceinline__ int block_argmax(const tv_t *logits, int n, uint32_t tag, CT &c, float *scr, int *anynan) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -INFINITY;
    int bi = -1, nan = 0;
    float vals[NA];
    const int cnt = n > tid ? (n - tid + kEngThreads - 1) / kEngThreads : 0;
    wait_strided<NA>(logits + tid, kEngThreads, cnt, tag, vals, c);
#pragma unroll
    for (int k = 0; k < NA; k++) {
        if (k >= cnt) continue;
        const int i = tid + k * kEngThreads;
        const float v = vals[k];
        if (v != v)
            nan = 1;
        else if (bi < 0 || v >= bv) {
            bv = v;
            bi = i;
        }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
            bv = ov;
            bi = oi;
        }
    }
    int *si = reinterpret_cast<int *>(scr);
    float *sv = scr + kEngWaves;
    *anynan = __syncthreads_or(nan);
    if (lane == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    float b = -INFINITY;
    int ix = -1;
#pragma unroll
    for (int w = 0; w < kEngWaves; w++)
        if (si[w] >= 0 && (ix < 0 || sv[w] > b || (sv[w] == b && si[w] > ix))) {
            b = sv[w];
            ix = si[w];
        }
    return ix;
}

// ---------------------------------------------------------------------------
// GEMV task: a slice of C output columns (C = 32, 16, 8 or 4 of a 32-column
// panel; for SwiGLU the same slice of the gate and the up panel) x one K
// chunk x M rows.  The host picks the narrowest slice that keeps the op
// within one task per block, so every GEMV spreads over the whole grid.
// Same arithmetic as k_gemv: acc += (scale * x) * nib - 8 * (scale * x), f32.
// ---------------------------------------------------------------------------
template <int M, int NP, int C, int R, class CT>
__device__ __forceinline__ int eng_gemv(const KCONST EngGemv &g, int task, uint32_t tb, CT &c, float *smem, int row) {
    constexpr int DW = q4_slice_dwords<C>();
    float *red = smem;                          // [NP][M][kEngWaves][C]
    float *scr = red + NP * M * kEngWaves * C;  // [M][kEngWaves] per-wave sums of squares
    float *sxr = scr + M * kEngWaves;           // [NP][M][kEngWaves] per-wave sums of scale * x
    const int tid = threadIdx.x;
    const int N = g.w.N, K = g.w.K;
    const int Nout = N / NP;
    const int P = Nout / 32;          // panels per half
    const int per_chunk = Nout / C;   // tasks per K chunk
    const int nonowner = per_chunk * (g.kc - 1);
    int tt, ch;
    if (task < nonowner) {
        tt = task % per_chunk;
        ch = 1 + task / per_chunk;
    } else {
        tt = task - nonowner;
        ch = 0;
    }
    // Slice-major: the slices of panel p are tasks p, p + P, ..., which run
    // on blocks P apart -- one XCD when P % 8 == 0 (blocks are dealt to the
    // 8 XCDs round-robin) -- so a panel's rows are fetched into one L2.
    const int p = tt % P, sl = tt / P;
    const int col0 = p * 32 + sl * C;  // first output column of the slice
    const int k0 = ch * g.kchunk;
    const int k1 = min(K, k0 + g.kchunk);
    int panel[NP];
    panel[0] = p;
    if (NP == 2) panel[NP - 1] = p + P;

    // 1. this chunk's weight rows, issued back to back before any input
    //    wait: row iterations are wave-uniform (nit), a thread past the
    //    chunk's last row re-reads that row (its input is zero), and the raw
    //    scale/gamma bits stay opaque until the accumulation, so no load
    //    result is needed (and waited for) while the others are issued.
    const int nit = (k1 - k0 + kEngThreads - 1) / kEngThreads;  // <= R
    const uint8_t *wq = reinterpret_cast<const uint8_t *>(g.w.wq) + sl * (C / 2);
    uint32_t wv[NP][R][DW];
    uint32_t sv[NP][R];
    uint32_t gam[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int k = min(k0 + tid + i * kEngThreads, k1 - 1);
#pragma unroll
        for (int pp = 0; pp < NP; pp++) {
#pragma unroll
            for (int d = 0; d < DW; d++) wv[pp][i][d] = 0u;
            sv[pp][i] = 0u;
            if (i < nit) {
                q4_slice_load<C>(wq + ((size_t)panel[pp] * K + k) * 16, wv[pp][i]);
                sv[pp][i] = __builtin_nontemporal_load(glb(g.w.ws) + (size_t)panel[pp] * K + k);
            }
        }
        gam[i] = 0u;
        if (g.norm && i < nit) gam[i] = glb(g.gamma)[k];
    }
    // The owner's bias and residual, also loaded before any wait.  The
    // residual is older than the input in the dependency chain and usually
    // complete by now (its tag is checked in the epilogue, which re-reads
    // it if not); loaded here, it does not sit in the queue behind the
    // input polls.
    const bool epi_lane = ch == 0 && NP == 1 && tid < M * C;
    float e_bias = 0.0f;
    uint64_t e_res = 0, e_res2 = 0;
    const tv_t *res_at = g.resid + (size_t)(tid / C + row) * g.ld_resid + col0 + (tid % C);  // EEPI_RESID without a table
    if (epi_lane && g.bias) e_bias = glb(g.bias)[col0 + (tid % C)];
    if (epi_lane && g.epi == EEPI_RESID) e_res = ld_dev_u64(g.resid_table ? g.resid_code : res_at);
    if (epi_lane && g.epi == EEPI_RESID && g.resid_parts == 2) e_res2 = ld_dev_u64(res_at + N);

    // The epilogue's plan for this lane, read out of the descriptor now
    // (while the loads fly) and held in vector registers: under SGPR
    // pressure the compiler would otherwise re-read each field after the
    // reduction, one dependent scalar-cache round trip per branch on the
    // critical path.  Flags: 1 norm, 2 second part of a split_out output,
    // 4 split-K partial, 8 owner waits for partials, 16 bias, 32 residual,
    // 64 residual from the table, 128 two-part residual, 256 plain copy,
    // 512 the normed input row is stored.
    const int e_m = tid / C + row, e_col = col0 + (tid % C);
    const bool e_second = ch > 0 && NP == 1 && g.split_out;
    uint32_t e_flags = (g.norm ? 1u : 0u) | (e_second ? 2u : 0u) | (ch > 0 && !e_second ? 4u : 0u) |
                       (ch == 0 && g.kc > 1 && !(NP == 1 && g.split_out) ? 8u : 0u) | (g.bias ? 16u : 0u) |
                       (g.epi == EEPI_RESID ? 32u : 0u) | (g.resid_table ? 64u : 0u) |
                       (g.resid_parts == 2 ? 128u : 0u) | (g.out_plain ? 256u : 0u) |
                       (g.norm_plain && tt == 0 && ch == 0 && row + M == g.M ? 512u : 0u);
    uint64_t e_dst = (uint64_t)(e_second ? g.out + (size_t)e_m * g.ld_out + N + e_col
                                : ch > 0 ? g.part + ((size_t)(ch - 1) * g.M + e_m) * N + e_col
                                         : g.out + (size_t)e_m * g.ld_out + e_col);
    uint32_t e_tag = tb + (ch > 0 && !e_second ? g.part_tag : g.out_tag);
    uint64_t e_part = (uint64_t)(g.part + (size_t)e_m * N + e_col);  // the owner's partials, stride M * N
    uint32_t e_pstride = (uint32_t)(g.M * N), e_nparts = (uint32_t)(g.kc - 1), e_ptag = tb + g.part_tag;
    uint64_t e_plain = (uint64_t)(g.out_plain + (size_t)e_m * g.ld_plain + e_col);
    uint64_t e_nplain = (uint64_t)g.norm_plain;
    uint32_t e_rtag = tb + g.resid_tag;
    float e_K = (float)K;
    asm volatile("" : "+v"(e_flags), "+v"(e_dst), "+v"(e_tag), "+v"(e_part), "+v"(e_pstride), "+v"(e_nparts));
    asm volatile("" : "+v"(e_ptag), "+v"(e_plain), "+v"(e_nplain), "+v"(e_rtag), "+v"(e_K));

    stamp(c, 2);
    // 2. inputs of this thread's rows.
    stamp(c, 3);
    float xv[R][M];
    float ssq[M];  // this thread's share of the row's sum of squares (norm only)
#pragma unroll
    for (int m = 0; m < M; m++) ssq[m] = 0.0f;
#pragma unroll
    for (int m = 0; m < M; m++) {
        const KCONST EngInput &in = g.in[m + row];
        if (in.kind == EIN_TV && g.norm) {
            // rms_norm_f16 (src/gemv.rs:406-417) over the full row, which is
            // this task's chunk (the host keeps normed GEMVs in one chunk of
            // <= 256 * kEngNormRows rows).
            constexpr int NR = R < kEngNormRows ? R : kEngNormRows;
#pragma unroll
            for (int i = 0; i < R; i++) asm volatile("" : "+v"(gam[i]));
            const int nj = K > tid ? (K - tid + kEngThreads - 1) / kEngThreads : 0;  // <= NR
            float row[NR];
            if (in.parts == 2) {
                // the two parts of a split_out output (nj <= NR / 2): a wider
                // poll (three parts of 2048) costs the whole kernel registers
                constexpr int H = NR / 2 > 0 ? NR / 2 : 1;
                float two[H];
                wait_pair<H>(in.tv + tid, in.tv + K + tid, kEngThreads, nj, tb + in.tag, two, c);
#pragma unroll
                for (int j = 0; j < NR; j++) row[j] = j < H ? two[j < H ? j : 0] : 0.0f;
            } else {
                wait_strided<NR>(in.tv + tid, kEngThreads, nj, tb + in.tag, row, c);
            }
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < NR; j++)
                if (j < nj) ss += row[j] * row[j];
            // The row is accumulated as x * gamma and the sums are scaled by
            // 1 / rms once the block's sum of squares is known (after the
            // reduction barrier), so no barrier sits before the accumulation.
            ssq[m] = ss;
#pragma unroll
            for (int i = 0; i < R; i++) xv[i][m] = i < NR && i < nj ? row[i < NR ? i : 0] * f16_to_f32((uint16_t)gam[i]) : 0.0f;
        } else if (in.kind == EIN_ARGTAB) {
            if constexpr (M == 1 && NP == 1) {
                // The row of a per-code table at the argmax of the logits:
                // the previous step's code and the projection of its
                // embedding in one step (the host builds the table and keeps
                // such inputs normed, in one chunk, M == 1).
                constexpr int NR = R < kEngNormRows ? R : kEngNormRows;
#pragma unroll
                for (int i = 0; i < R; i++) asm volatile("" : "+v"(gam[i]));
                int anynan = 0;
                const int ix = block_argmax<kEngArgtabMax / kEngThreads>(in.tv, in.n, tb + in.tag, c,
                                                                        smem + kEngSmemFloats - 2 * kEngWaves, &anynan);
                const uint32_t tok = (ix < 0 || anynan) ? 0u : (uint32_t)ix;  // the argmax step's code
                const int nj = K > tid ? (K - tid + kEngThreads - 1) / kEngThreads : 0;  // <= NR
                const auto *trow = glb(in.table) + (size_t)(tok < (uint32_t)in.table_rows ? tok : 0u) * K + tid;
                const bool have = tok < (uint32_t)in.table_rows;
                float row[NR];
#pragma unroll
                for (int j = 0; j < NR; j++) row[j] = j < nj && have ? trow[j * kEngThreads] : 0.0f;
                float ss = 0.0f;
#pragma unroll
                for (int j = 0; j < NR; j++)
                    if (j < nj) ss += row[j] * row[j];
                ssq[m] = ss;
#pragma unroll
                for (int i = 0; i < R; i++)
                    xv[i][m] = i < NR && i < nj ? row[i < NR ? i : 0] * f16_to_f32((uint16_t)gam[i]) : 0.0f;
            }
        } else if (in.kind == EIN_TV) {
            const int cnt = k1 > k0 + tid ? (k1 - k0 - tid + kEngThreads - 1) / kEngThreads : 0;
            float row[R];
            wait_strided<R>(in.tv + k0 + tid, kEngThreads, cnt, tb + in.tag, row, c);
#pragma unroll
            for (int i = 0; i < R; i++) xv[i][m] = i < cnt ? row[i] : 0.0f;
        } else if (in.kind == EIN_PLAIN) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int k = k0 + tid + i * kEngThreads;
                xv[i][m] = k < k1 ? ld_dev(&in.plain[k]) : 0.0f;
            }
        } else {
            // embed_lookup_q4 (src/gemv.rs:377-400) of the tagged token's row.
            const uint32_t tok = wait_tv_u32(in.tok_tv, tb + in.tag, c);
            float ev[R];
#pragma unroll
            for (int i = 0; i < R; i++) ev[i] = 0.0f;
            if (tok < (uint32_t)in.emb.K) q4_gather<R>(in.emb, tok, k0 + tid, kEngThreads, k1, ev);
#pragma unroll
            for (int i = 0; i < R; i++) xv[i][m] = ev[i];
        }
    }

    // Every input value is final here: one wait, not one per row of the
    // accumulation below.
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int m = 0; m < M; m++) asm volatile("" : "+v"(xv[i][m]));
    // A residual read before it was complete (a block that ran ahead) is
    // read again now; the load flies during the accumulation.
    float e_tab = 0.0f;  // the residual read from resid_table
    if (epi_lane && g.epi == EEPI_RESID && g.resid_table) {
        const uint32_t code = (uint32_t)(e_res >> 32) == e_rtag ? (uint32_t)e_res : wait_tv_u32(g.resid_code, e_rtag, c);
        if (code < (uint32_t)g.resid_table_rows) e_tab = glb(g.resid_table)[(size_t)code * g.ld_resid + col0 + (tid % C)];
    } else if (epi_lane && g.epi == EEPI_RESID) {
        if ((uint32_t)(e_res >> 32) != e_rtag) e_res = ld_dev_u64(res_at);
        if (g.resid_parts == 2 && (uint32_t)(e_res2 >> 32) != e_rtag) e_res2 = ld_dev_u64(res_at + N);
    }
    stamp(c, 4);
    // 3. accumulate the slice's columns per panel.
    float acc[NP][M][C];
#pragma unroll
    for (int pp = 0; pp < NP; pp++)
#pragma unroll
        for (int m = 0; m < M; m++)
#pragma unroll
            for (int j = 0; j < C; j++) acc[pp][m][j] = 0.0f;
    // weights and scales are consumed only from here on
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int pp = 0; pp < NP; pp++) {
            asm volatile("" : "+v"(sv[pp][i]));
#pragma unroll
            for (int d = 0; d < DW; d++) asm volatile("" : "+v"(wv[pp][i][d]));
        }
    // Each term is (scale * x) * nib - 8 * (scale * x): the offset is applied
    // once per column, after the reduction, from the block's sum of
    // scale * x, kept (like the products' operands) scaled by 2^24.
    float sxsum[NP][M];
#pragma unroll
    for (int pp = 0; pp < NP; pp++)
#pragma unroll
        for (int m = 0; m < M; m++) sxsum[pp][m] = 0.0f;
#pragma unroll
    for (int i = 0; i < R; i++) {
        if (i >= nit) continue;  // uniform; rows past k1 carry a zero input
        float xa[M];
#pragma unroll
        for (int m = 0; m < M; m++) xa[m] = xv[i][m] * 16777216.0f;
#pragma unroll
        for (int pp = 0; pp < NP; pp++) {
            const float s = f16_to_f32((uint16_t)sv[pp][i]);
            float sa[M], sb[M];
#pragma unroll
            for (int m = 0; m < M; m++) {
                sa[m] = s * xa[m];
                sb[m] = sa[m] * 0.0625f;
                sxsum[pp][m] += sa[m];
            }
            q4_mix_row<M, C>(wv[pp][i], sa, sb, acc[pp]);
        }
    }

    stamp(c, 5);
    // 4. block reduction (lane exchanges within each wave, then the waves
    //    through LDS).  Thread (m, j) < M * C ends with column j of row m of
    //    every panel, so the split-K exchange and the epilogue stay in its
    //    registers.
#pragma unroll
    for (int pp = 0; pp < NP; pp++)
#pragma unroll
        for (int m = 0; m < M; m++) {
            if constexpr (C == 32)
                lane_reduce32(acc[pp][m], &red[(pp * M + m) * kEngWaves * C]);
            else if constexpr (C == 16)
                lane_reduce16(acc[pp][m], &red[(pp * M + m) * kEngWaves * C]);
            else
                dpp_reduce<C>(acc[pp][m], &red[(pp * M + m) * kEngWaves * C]);
            const float w = wave_sum(sxsum[pp][m]);
            if ((tid & 63) == 0) sxr[(pp * M + m) * kEngWaves + (tid >> 6)] = w;
        }
    if (g.norm) {
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float w = wave_sum(ssq[m]);
            if ((tid & 63) == 0) scr[kEngWaves * m + (tid >> 6)] = w;
        }
    }
    __syncthreads();
    stamp(c, 6);
    // 1 / rms of input row m (rms_norm_f16, src/gemv.rs:406-417), computed
    // only by the lanes that use it
    auto inv_of = [&](int m) { return 1.0f / sqrtf(waves_sum(&scr[kEngWaves * m], 1) / e_K + 1e-6f); };
    const uint32_t fl = __builtin_amdgcn_readfirstlane(e_flags);  // uniform
    if (fl & 512u) {
        // the normed last row, for a later launch
        const float iv = inv_of(M - 1);
        float *np_row = reinterpret_cast<float *>(e_nplain);
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int k = k0 + tid + i * kEngThreads;
            if (i < nit && k < k1) st_dev(&np_row[k], xv[i][M - 1] * iv);
        }
    }
    if (tid < M * C) {
        const int m = tid / C, j = tid % C;
        float y[NP];
#pragma unroll
        for (int pp = 0; pp < NP; pp++) {
            y[pp] = fmaf(-0x1p-21f, waves_sum(&sxr[(pp * M + m) * kEngWaves], 1),
                         waves_sum(&red[(pp * M + m) * kEngWaves * C + j], C));
        }
        // 5. split-K: non-owners publish partials; the owner adds them in order.
        tv_t *dst = reinterpret_cast<tv_t *>(e_dst);
        if (fl & 2u) {  // the second part of a split_out output
            put_tv(dst, y[0], e_tag);
            return -1;
        }
        if (fl & 4u) {
#pragma unroll
            for (int pp = 0; pp < NP; pp++) put_tv(dst + pp * Nout, y[pp], e_tag);
            return -1;
        }
        if (fl & 8u) {
#pragma unroll
            for (int pp = 0; pp < NP; pp++) {
                float pv4[4];
                wait_strided<4>(reinterpret_cast<const tv_t *>(e_part) + pp * Nout, e_pstride, (int)e_nparts, e_ptag,
                                pv4, c);
#pragma unroll
                for (int cc = 0; cc < 4; cc++)
                    if (cc < (int)e_nparts) y[pp] += pv4[cc];
            }
        }
        if (fl & 1u) {
            const float iv = inv_of(m);
#pragma unroll
            for (int pp = 0; pp < NP; pp++) y[pp] *= iv;
        }
        // 6. epilogue
        if (NP == 2) {
            // silu(g) * u, src/talker.rs:342-345
            const float gt = y[0], up = y[NP - 1];
            put_tv(dst, (gt / (1.0f + expf(-gt))) * up, e_tag);
        } else {
            float v = y[0];
            if (fl & 16u) v += e_bias;
            if (fl & 32u) {
                float r;
                if (fl & 64u) {
                    r = e_tab;
                } else {
                    r = (uint32_t)(e_res >> 32) == e_rtag ? __uint_as_float((uint32_t)e_res) : wait_tv(res_at, e_rtag, c);
                    if (fl & 128u)
                        r += (uint32_t)(e_res2 >> 32) == e_rtag ? __uint_as_float((uint32_t)e_res2)
                                                                : wait_tv(res_at + N, e_rtag, c);
                }
                v = r + v;
            }
            put_tv(dst, v, e_tag);
            if (fl & 256u) st_dev(reinterpret_cast<float *>(e_plain), v);
        }
    }
    if (ch > 0) return -1;
    stamp(c, 7);
    return col0;
}

template <int M, int NP, class CT>
__device__ __forceinline__ int eng_gemv_cols(const KCONST EngGemv &g, int task, uint32_t tb, CT &c, float *smem, int row) {
    // Whole 32-column panels: narrower slices spread an op over more blocks
    // but leave fewer blocks idle to run ahead into the next op (issuing its
    // weight loads early), which costs more than the shorter accumulation
    // saves on this loop -- except for the SwiGLU step when its half-panel
    // tasks still fit the grid (the host's choice): that task is the
    // heaviest (two panels and two reductions).
    if constexpr (NP == 2)
        if (g.cols == 16) return eng_gemv<M, 2, 16, eng_rows_per_thread(16, 2)>(g, task, tb, c, smem, row);
    return eng_gemv<M, NP, 32, eng_rows_per_thread(32, NP)>(g, task, tb, c, smem, row);
}

// ---------------------------------------------------------------------------
// Attention task: one kv head x one split of positions, M query rows.
// QK-norm (src/talker.rs:86-99) and split-half RoPE (src/rope.rs:79-92) of the
// raw q/k, K/V append (src/talker.rs:299-302), then softmax(q.K^T*scale).V
// over the split (src/talker.rs:304-331), causal across the M new rows.
// ---------------------------------------------------------------------------
// NPI: (row, head) pairs rounded up; KJ: positions per thread held in
// registers for the scores (16 lanes each, NSLOT = kEngThreads / 16 positions
// at a time) -- a register batch covers PB = NSLOT * KJ positions.
template <int NPI, int KJ, class CT>
__device__ __forceinline__ int eng_attn_t(const KCONST EngAttn &a, int task, uint32_t tb, const EngState &st, CT &c,
                                          float *smem) {
    constexpr int HD = 128, HALF = 64, CH = 256;
    constexpr int NSLOT = kEngThreads / 16;  // positions per score round (16 lanes each)
    constexpr int NR8 = kEngThreads / 32;    // P.V position groups (32 lanes of 4 dims each)
    constexpr int PB = NSLOT * KJ;           // positions per register batch
    constexpr int VJ = PB / NR8;             // positions per thread for P.V
    static_assert(PB <= CH, "a register batch must fit the score buffer");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.nq / a.nkv;
    const int M = a.M;
    const int npi = M * G;  // (row, head) pairs, <= NPI
    const int kvh = task / a.nsplit, sp = task - kvh * a.nsplit;
    const int base = a.from_state ? st.kvlen : a.len_const;
    const int pos0 = a.from_state ? st.pos : a.pos_const;
    const int Lt = base + M;
    const int chunk = (Lt + a.nsplit - 1) / a.nsplit;
    const int t0 = sp * chunk, t1 = min(Lt, t0 + chunk);
    const int nt = max(0, t1 - t0);      // <= CH
    float *qs = smem;                    // [M][G][HD]
    float *kn = qs + kEngMaxM * 4 * HD;  // [M][HD]
    float *vn = kn + kEngMaxM * HD;      // [M][HD]
    float *sc = vn + kEngMaxM * HD;      // [NPI][CH] scores
    float *pt = sc + kEngMaxM * 4 * CH;  // [CH][NPI] probabilities (position-major)
    float *ml = pt + kEngMaxM * 4 * CH;  // [NPI][2]
    float *pvb = ml + 16;                // [kEngWaves][NPI][HD] P.V partials
    float *Kb = a.kcache + (size_t)kvh * a.kv_cap * HD;
    float *Vb = a.vcache + (size_t)kvh * a.kv_cap * HD;
    const int l16 = tid & 15, slot = tid >> 4;  // scores: 16 lanes per position, 8 dims per lane
    const int d4 = tid & 31, r8 = tid >> 5;     // P.V: 4 dims, every NR8-th position

    // Cached rows [0, base) for the register batch starting at position b0.
    // from_state: the rows were written by earlier launches, so plain loads
    // see them and may be issued before this step's inputs arrive.
    // Otherwise (rows appended earlier in this launch, possibly on another
    // XCD) they are read device-coherently after the inputs.  Positions past
    // the split read as zero.
    u32x4 kr[KJ][2];
    u32x4 vr[VJ];
    const u32x4 z4 = (u32x4){0u, 0u, 0u, 0u};
    auto load16 = [&](const float *p) -> u32x4 {
        if (a.from_state) return glb(reinterpret_cast<const u32x4 *>(p))[0];
        const uint64_t *q = reinterpret_cast<const uint64_t *>(p);
        const uint64_t e0 = ld_dev_u64(q), e1 = ld_dev_u64(q + 1);
        return (u32x4){(uint32_t)e0, (uint32_t)(e0 >> 32), (uint32_t)e1, (uint32_t)(e1 >> 32)};
    };
    auto load_k = [&](int b0) {
#pragma unroll
        for (int j = 0; j < KJ; j++) {
            const int tt = b0 + slot + NSLOT * j, t = t0 + tt;
            kr[j][0] = kr[j][1] = z4;
            if (tt < nt && t < base) {
                const float *src = Kb + (size_t)t * HD + l16 * 8;
                kr[j][0] = load16(src);
                kr[j][1] = load16(src + 4);
            }
        }
    };
    auto load_v = [&](int b0) {
#pragma unroll
        for (int u = 0; u < VJ; u++) {
            const int tt = b0 + r8 + NR8 * u, t = t0 + tt;
            vr[u] = z4;
            if (tt < nt && t < base) vr[u] = load16(Vb + (size_t)t * HD + 4 * d4);
        }
    };
    // the M new rows of the batch come from LDS
    auto patch_k = [&](int b0) {
#pragma unroll
        for (int j = 0; j < KJ; j++) {
            const int tt = b0 + slot + NSLOT * j, t = t0 + tt;
            if (tt < nt && t >= base) {
                kr[j][0] = *reinterpret_cast<const u32x4 *>(&kn[(t - base) * HD + l16 * 8]);
                kr[j][1] = *reinterpret_cast<const u32x4 *>(&kn[(t - base) * HD + l16 * 8 + 4]);
            }
        }
    };
    auto patch_v = [&](int b0) {
#pragma unroll
        for (int u = 0; u < VJ; u++) {
            const int tt = b0 + r8 + NR8 * u, t = t0 + tt;
            if (tt < nt && t >= base) vr[u] = *reinterpret_cast<const u32x4 *>(&vn[(t - base) * HD + 4 * d4]);
        }
    };

    // 0. inputs that do not depend on this step: norm gammas, RoPE rows, and
    //    (from_state) the first batch of cached K/V.
    const float gq1 = f16_to_f32(glb(a.q_norm)[lane]), gq2 = f16_to_f32(glb(a.q_norm)[lane + HALF]);
    const float gk1 = f16_to_f32(glb(a.k_norm)[lane]), gk2 = f16_to_f32(glb(a.k_norm)[lane + HALF]);
    float rcs[kEngMaxM], rsn[kEngMaxM];
    bool rok[kEngMaxM];
#pragma unroll
    for (int m = 0; m < kEngMaxM; m++) {
        const int pos = pos0 + m;
        rok[m] = m < M && !(a.rope_skip_oob && pos >= a.rope_rows);
        rcs[m] = rok[m] ? glb(a.rope_cos)[(size_t)pos * HALF + lane] : 1.0f;
        rsn[m] = rok[m] ? glb(a.rope_sin)[(size_t)pos * HALF + lane] : 0.0f;
    }
    if (a.from_state) {
        load_k(0);
        load_v(0);
    }
    stamp(c, 2);

    // 1. raw q (G heads), k, v of this kv head for the M rows
    const int per = (G + 2) * HD;
    {
        constexpr int NB = kEngMaxM * 6 * HD / kEngThreads;  // M <= 2, G <= 4
        const tv_t *ptr[NB];
        uint32_t tg[NB];
        float val[NB];
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int idx = tid + i * kEngThreads;
            tg[i] = tb + a.qkv_tag;
            ptr[i] = a.qkv;
            if (idx < M * per) {
                const int m = idx / per, r = idx - m * per, prt = r / HD, dd = r - prt * HD;
                int src;
                if (prt < G)
                    src = (kvh * G + prt) * HD + dd;
                else if (prt == G)
                    src = a.nq * HD + kvh * HD + dd;
                else
                    src = (a.nq + a.nkv) * HD + kvh * HD + dd;
                ptr[i] = &a.qkv[(size_t)m * a.ld_qkv + src];
                cnt = i + 1;
            }
        }
        wait_list<NB>(ptr, tg, cnt, val, c);
        if (!a.from_state) {
            load_k(0);
            load_v(0);
        }
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int idx = tid + i * kEngThreads;
            if (idx >= M * per) continue;
            const int m = idx / per, r = idx - m * per, prt = r / HD, dd = r - prt * HD;
            if (prt < G)
                qs[(m * G + prt) * HD + dd] = val[i];
            else if (prt == G)
                kn[m * HD + dd] = val[i];
            else
                vn[m * HD + dd] = val[i];
        }
    }
    __syncthreads();
    stamp(c, 3);
    // 2. QK-norm (src/talker.rs:86-99) + split-half RoPE (src/rope.rs:79-92), one wave per vector
    for (int vi = wave; vi < M * (G + 1); vi += kEngWaves) {
        const int m = vi / (G + 1), r = vi - m * (G + 1);
        float *vec = r < G ? &qs[(m * G + r) * HD] : &kn[m * HD];
        const float x1 = vec[lane], x2 = vec[lane + HALF];
        const float ss = wave_sum(x1 * x1 + x2 * x2);
        const float inv = 1.0f / sqrtf(ss / (float)HD + 1e-6f);
        const float n1 = x1 * inv * (r < G ? gq1 : gk1);
        const float n2 = x2 * inv * (r < G ? gq2 : gk2);
        const float cs = m == 0 ? rcs[0] : rcs[kEngMaxM - 1], sn = m == 0 ? rsn[0] : rsn[kEngMaxM - 1];
        const bool rp = m == 0 ? rok[0] : rok[kEngMaxM - 1];
        vec[lane] = rp ? n1 * cs - n2 * sn : n1;
        vec[lane + HALF] = rp ? n2 * cs + n1 * sn : n2;
    }
    __syncthreads();
    stamp(c, 4);
    // 3. append the new rows that fall in this split (src/talker.rs:299-302)
    for (int idx = tid; idx < M * HD; idx += kEngThreads) {
        const int m = idx / HD, dd = idx - m * HD, t = base + m;
        if (t >= t0 && t < t1) {
            st_dev(&Kb[(size_t)t * HD + dd], kn[m * HD + dd]);
            st_dev(&Vb[(size_t)t * HD + dd], vn[m * HD + dd]);
        }
    }
    // q of this lane's 8 dims, per (row, head)
    float q8[NPI][8];
#pragma unroll
    for (int pi = 0; pi < NPI; pi++)
#pragma unroll
        for (int e = 0; e < 8; e++) q8[pi][e] = pi < npi ? qs[pi * HD + l16 * 8 + e] : 0.0f;
    stamp(c, 5);
    // 4. scores q.K^T * scale, causal across the M new rows (src/talker.rs:304-318)
    for (int b0 = 0; b0 < nt; b0 += PB) {
        if (b0 > 0) load_k(b0);
        patch_k(b0);
#pragma unroll
        for (int j = 0; j < KJ; j++) {
            const int tt = b0 + slot + NSLOT * j, t = t0 + tt;
            const float k8[8] = {__uint_as_float(kr[j][0].x), __uint_as_float(kr[j][0].y), __uint_as_float(kr[j][0].z),
                                 __uint_as_float(kr[j][0].w), __uint_as_float(kr[j][1].x), __uint_as_float(kr[j][1].y),
                                 __uint_as_float(kr[j][1].z), __uint_as_float(kr[j][1].w)};
#pragma unroll
            for (int pi = 0; pi < NPI; pi++) {
                float dot = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) dot += q8[pi][e] * k8[e];
                dot = row16_sum(dot);
                const int m = pi / G;
                if (l16 == 0 && pi < npi && tt < min(nt, b0 + PB))
                    sc[pi * CH + tt] = (t <= base + m) ? dot * a.scale : -INFINITY;
            }
        }
    }
    __syncthreads();
    stamp(c, 6);
    // 5. local softmax statistics, one wave per (row, head) (src/talker.rs:319-326);
    //    the probabilities go to pt position-major, zero past the split.
    const int ntp = (nt + PB - 1) / PB * PB;  // P.V reads whole batches
    for (int pi = wave; pi < NPI; pi += kEngWaves) {
        if (pi >= npi) {
            for (int t = lane; t < ntp; t += 64) pt[t * NPI + pi] = 0.0f;
            continue;
        }
        float mx = -INFINITY;
        for (int t = lane; t < nt; t += 64) mx = fmaxf(mx, sc[pi * CH + t]);
        mx = wave_max(mx);
        float l = 0.0f;
        for (int t = lane; t < ntp; t += 64) {
            float e = 0.0f;
            if (t < nt) {
                const float s = sc[pi * CH + t];
                e = (mx == -INFINITY) ? 0.0f : expf(s - mx);
            }
            pt[t * NPI + pi] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            ml[pi * 2] = mx;
            ml[pi * 2 + 1] = l;
        }
    }
    __syncthreads();
    stamp(c, 7);
    // 6. P.V (src/talker.rs:327-331): thread (4 dims, position group) over
    //    its positions; the NR8 groups are added by a lane swap across the
    //    wave halves and then through LDS.
    {
        float acc[NPI][4];
#pragma unroll
        for (int pi = 0; pi < NPI; pi++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[pi][e] = 0.0f;
        for (int b0 = 0; b0 < nt; b0 += PB) {
            if (b0 > 0 || nt > PB) load_v(b0);  // a single-batch split reuses the early loads
            patch_v(b0);
#pragma unroll
            for (int u = 0; u < VJ; u++) {
                const int tt = b0 + r8 + NR8 * u;
                float p[NPI];
                if (NPI == 2) {
                    const float2 q = *reinterpret_cast<const float2 *>(&pt[tt * NPI]);
                    p[0] = q.x;
                    p[NPI - 1] = q.y;
                } else {
#pragma unroll
                    for (int h4 = 0; h4 < NPI / 4; h4++) {
                        const float4 q = *reinterpret_cast<const float4 *>(&pt[tt * NPI + 4 * h4]);
                        p[4 * h4] = q.x;
                        p[4 * h4 + 1] = q.y;
                        p[4 * h4 + 2] = q.z;
                        p[4 * h4 + 3] = q.w;
                    }
                }
                const float v[4] = {__uint_as_float(vr[u].x), __uint_as_float(vr[u].y), __uint_as_float(vr[u].z),
                                    __uint_as_float(vr[u].w)};
#pragma unroll
                for (int pi = 0; pi < NPI; pi++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[pi][e] += p[pi] * v[e];
            }
        }
#pragma unroll
        for (int pi = 0; pi < NPI; pi++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[pi][e] = halves_sum(acc[pi][e]);
        if (lane < 32) {
#pragma unroll
            for (int pi = 0; pi < NPI; pi++)
                *reinterpret_cast<float4 *>(&pvb[(wave * NPI + pi) * HD + 4 * d4]) =
                    make_float4(acc[pi][0], acc[pi][1], acc[pi][2], acc[pi][3]);
        }
        // Rows appended in this launch are read by later steps of the same
        // launch: their stores complete before the outputs that order those
        // steps.  Rows of a from_state step are only read by later launches.
        if (!a.from_state) wait_stores();
        __syncthreads();
        for (int idx = tid; idx < npi * HD; idx += kEngThreads) {
            const int pi = idx / HD, d = idx - pi * HD;
            const int m = pi / G, g = pi - m * G, h = kvh * G + g;
            const float o = waves_sum(&pvb[pi * HD + d], NPI * HD);
            if (a.nsplit == 1) {
                const float l = ml[pi * 2 + 1];
                put_tv(&a.out[(size_t)m * a.nq * HD + h * HD + d], o / l, tb + a.out_tag);
            } else {
                tv_t *dst = a.part + (((size_t)m * a.nq + h) * a.nsplit + sp) * (HD + 2);
                put_tv(&dst[2 + d], o, tb + a.part_tag);
                if (d == 0) {
                    put_tv(&dst[0], ml[pi * 2], tb + a.part_tag);
                    put_tv(&dst[1], ml[pi * 2 + 1], tb + a.part_tag);
                }
            }
        }
    }
    return task;
}

// ---------------------------------------------------------------------------
// Short in-launch attention (the predictor: <= 32 positions, one kv head
// per task).  Every step of a layer runs task h on the same block, so the
// rows of kv head h appended by earlier steps of this launch are in that
// block's LDS (lds_kv), and one wave per (row, q head) works without a block
// barrier.  Lane l holds dims 2l, 2l+1 of every vector; RoPE pairs
// (d, d+64) sit 32 lanes apart (v_permlane32_swap).  Scores are reduced over
// the wave by lane exchanges, softmax runs across lanes (one position each)
// and P.V takes the probabilities by readlane.  Same arithmetic as
// eng_attn_t: QK-norm (src/talker.rs:86-99), split-half RoPE
// (src/rope.rs:79-92), softmax(q.K^T*scale).V with the sum divided out at
// the end (src/talker.rs:304-331), causal across the M new rows.  The rows
// are also written to the device cache, for the host.
// ---------------------------------------------------------------------------
template <class CT>
__device__ __forceinline__ int eng_attn_lean(const KCONST EngAttn &a, int task, uint32_t tb, CT &c, float *smem,
                                             float *kvl) {
    constexpr int HD = 128, HALF = 64, NP = kEngLdsKvPos;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches below
    const int G = a.nq / a.nkv;
    const int M = a.M;
    uint32_t tcode = 0;  // qkv_table: the previous step's code, taken by the whole block
    if (a.qkv_table) {
        int anynan = 0;
        const int ix = block_argmax<kEngArgtabMax / kEngThreads>(a.logits, a.logits_n, tb + a.logits_tag, c,
                                                                smem + kEngSmemFloats - 2 * kEngWaves, &anynan);
        tcode = (ix < 0 || anynan) ? 0u : (uint32_t)ix;
    }
    if (wave >= M * G) return task;
    const int m = wave / G, gq = wave - m * G, kvh = task, h = kvh * G + gq;
    const int base = a.len_const, pos0 = a.pos_const;
    const int nvis = base + m + 1;  // positions row m attends to
    const int d0 = 2 * lane;        // this lane's dims d0, d0 + 1
    const int i0 = d0 & (HALF - 1);  // their RoPE table index
    float *Kl = kvl + d0, *Vl = kvl + NP * HD + d0;  // row t of this lane: Kl[t * HD]

    // 0. step-independent inputs: gammas, RoPE rows
    const uint32_t gqb = glb(reinterpret_cast<const uint32_t *>(a.q_norm))[lane];
    const uint32_t gkb = glb(reinterpret_cast<const uint32_t *>(a.k_norm))[lane];
    float rc[kEngMaxM][2], rs[kEngMaxM][2];
#pragma unroll
    for (int r = 0; r < kEngMaxM; r++) {
        const int pos = pos0 + r;
        rc[r][0] = rc[r][1] = 1.0f;
        rs[r][0] = rs[r][1] = 0.0f;
        if (r < M && !(a.rope_skip_oob && pos >= a.rope_rows)) {
            const uint64_t cb = glb(reinterpret_cast<const uint64_t *>(a.rope_cos + (size_t)pos * HALF + i0))[0];
            const uint64_t sb = glb(reinterpret_cast<const uint64_t *>(a.rope_sin + (size_t)pos * HALF + i0))[0];
            rc[r][0] = __uint_as_float((uint32_t)cb);
            rc[r][1] = __uint_as_float((uint32_t)(cb >> 32));
            rs[r][0] = __uint_as_float((uint32_t)sb);
            rs[r][1] = __uint_as_float((uint32_t)(sb >> 32));
        }
    }
    stamp(c, 2);

    // 1. raw q of (row m, head h), k and v of the M new rows
    constexpr int NW = 2 + 4 * kEngMaxM;
    const tv_t *ptr[NW];
    uint32_t tg[NW];
    float val[NW];
    const size_t qoff = (size_t)h * HD + d0, koff = (size_t)(a.nq + kvh) * HD + d0,
                 voff = (size_t)(a.nq + a.nkv + kvh) * HD + d0;
#pragma unroll
    for (int i = 0; i < NW; i++) {
        tg[i] = tb + a.qkv_tag;
        ptr[i] = a.qkv;
    }
    ptr[0] = &a.qkv[(size_t)m * a.ld_qkv + qoff];
    ptr[1] = ptr[0] + 1;
#pragma unroll
    for (int r = 0; r < kEngMaxM; r++) {
        if (r >= M) continue;
        ptr[2 + 4 * r] = &a.qkv[(size_t)r * a.ld_qkv + koff];
        ptr[3 + 4 * r] = ptr[2 + 4 * r] + 1;
        ptr[4 + 4 * r] = &a.qkv[(size_t)r * a.ld_qkv + voff];
        ptr[5 + 4 * r] = ptr[4 + 4 * r] + 1;
    }
    if (a.qkv_table) {
        // one new row (M == 1): its raw q, k, v from the table row at the code
        const bool have = tcode < (uint32_t)a.qkv_table_rows;
        const float *row = a.qkv_table + (size_t)(have ? tcode : 0u) * a.ld_qkv;
        const uint64_t qb = glb(reinterpret_cast<const uint64_t *>(row + qoff))[0];
        const uint64_t kb = glb(reinterpret_cast<const uint64_t *>(row + koff))[0];
        const uint64_t vb = glb(reinterpret_cast<const uint64_t *>(row + voff))[0];
        val[0] = have ? __uint_as_float((uint32_t)qb) : 0.0f;
        val[1] = have ? __uint_as_float((uint32_t)(qb >> 32)) : 0.0f;
        val[2] = have ? __uint_as_float((uint32_t)kb) : 0.0f;
        val[3] = have ? __uint_as_float((uint32_t)(kb >> 32)) : 0.0f;
        val[4] = have ? __uint_as_float((uint32_t)vb) : 0.0f;
        val[5] = have ? __uint_as_float((uint32_t)(vb >> 32)) : 0.0f;
    } else {
        wait_list<NW>(ptr, tg, 2 + 4 * M, val, c);
    }
    stamp(c, 3);

    // 2. QK-norm + RoPE of q and of the new k rows
    const float gq0 = f16_to_f32((uint16_t)gqb), gq1 = f16_to_f32((uint16_t)(gqb >> 16));
    const float gk0 = f16_to_f32((uint16_t)gkb), gk1 = f16_to_f32((uint16_t)(gkb >> 16));
    // the first half (dims < 64) rotates as x c - x' s, the second as x c + x' s
    const float sgn = lane < 32 ? -1.0f : 1.0f;
    auto norm_rope = [&](float x0, float x1, float g0, float g1, int r, float &o0, float &o1) {
        const float inv = 1.0f / sqrtf(wave_sum(x0 * x0 + x1 * x1) / (float)HD + 1e-6f);
        const float n0 = x0 * inv * g0, n1 = x1 * inv * g1;
        const auto p0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(n0), __float_as_uint(n0), false, false);
        const auto p1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(n1), __float_as_uint(n1), false, false);
        // the value 32 lanes away: lanes < 32 get it in [1], lanes >= 32 in [0]
        const float q0 = __uint_as_float(lane < 32 ? p0[1] : p0[0]), q1 = __uint_as_float(lane < 32 ? p1[1] : p1[0]);
        const int ri = r == 0 ? 0 : kEngMaxM - 1;
        o0 = n0 * rc[ri][0] + sgn * (q0 * rs[ri][0]);
        o1 = n1 * rc[ri][1] + sgn * (q1 * rs[ri][1]);
    };
    float qn0, qn1;
    norm_rope(val[0], val[1], gq0, gq1, m, qn0, qn1);
    // 3. append the new rows (src/talker.rs:299-302) to the block's LDS,
    //    where this step reads them too (every wave of the task writes the
    //    same values before reading), and to the device cache
#pragma unroll
    for (int r = 0; r < kEngMaxM; r++) {
        if (r >= M) continue;
        float k0, k1;
        norm_rope(val[2 + 4 * r], val[3 + 4 * r], gk0, gk1, r, k0, k1);
        const float v0 = val[4 + 4 * r], v1 = val[5 + 4 * r];
        const int t = base + r;
        *reinterpret_cast<float2 *>(&Kl[t * HD]) = make_float2(k0, k1);
        *reinterpret_cast<float2 *>(&Vl[t * HD]) = make_float2(v0, v1);
        st_dev_u64(reinterpret_cast<uint64_t *>(a.kcache + ((size_t)kvh * a.kv_cap + t) * HD + d0),
                   ((uint64_t)__float_as_uint(k1) << 32) | __float_as_uint(k0));
        st_dev_u64(reinterpret_cast<uint64_t *>(a.vcache + ((size_t)kvh * a.kv_cap + t) * HD + d0),
                   ((uint64_t)__float_as_uint(v1) << 32) | __float_as_uint(v0));
    }
    stamp(c, 4);

    // 4. scores over positions t < nvis, reduced over the wave into
    //    red[wave][t]
    //    (all NP rows are read at once, so the reads are not serialised
    //    behind branches; columns past nvis hold stale or uninitialised rows
    //    and are masked in the softmax -- the reduction keeps columns apart)
    float2 kr[NP];
#pragma unroll
    for (int t = 0; t < NP; t++) kr[t] = *reinterpret_cast<const float2 *>(&Kl[t * HD]);
    float part[NP];
#pragma unroll
    for (int t = 0; t < NP; t++) part[t] = qn0 * kr[t].x + qn1 * kr[t].y;
    float *red = smem;  // [M * G waves][NP]
    static_assert(NP == 32, "the lean attention reduces 32 positions");
    lane_reduce32(part, red);
    // 5. softmax across lanes, position t on lane t
    const float sc = lane < nvis ? red[wave * NP + lane] * a.scale : -INFINITY;
    const float mx = wave_max(sc);
    const float e = lane < nvis ? expf(sc - mx) : 0.0f;
    const float l = wave_sum(e);
    stamp(c, 5);
    // 6. P.V
    float2 vr[NP];
#pragma unroll
    for (int t = 0; t < NP; t++) vr[t] = *reinterpret_cast<const float2 *>(&Vl[t * HD]);
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int t = 0; t < NP; t++) {
        if (t < nvis) {  // uniform
            const float pt = lane_f(e, t);
            o0 += pt * vr[t].x;
            o1 += pt * vr[t].y;
        }
    }
    tv_t *dst = &a.out[(size_t)m * a.nq * HD + (size_t)h * HD + d0];
    put_tv(dst, o0 / l, tb + a.out_tag);
    put_tv(dst + 1, o1 / l, tb + a.out_tag);
    stamp(c, 6);
    return task;
}

template <class CT>
__device__ __forceinline__ int eng_attn(const KCONST EngAttn &a, int task, uint32_t tb, const EngState &st, CT &c,
                                        float *smem, float *kvl) {
    if (a.lds_kv) return eng_attn_lean(a, task, tb, c, smem, kvl);
    const int npi = a.M * (a.nq / a.nkv);
    const int Lt = (a.from_state ? st.kvlen : a.len_const) + a.M;
    const bool small = (Lt + a.nsplit - 1) / a.nsplit <= kEngThreads / 16;
    // at most two (row, head) pairs (the host runs other shapes on the
    // multi-kernel path; wider instantiations cost the whole kernel registers).
    // A register batch of 64 positions holds a talker split of capacity / 48
    // rows whole; longer splits (over 32 splits' worth of cache) take more
    // batches.
    if (npi <= 2) return small ? eng_attn_t<2, 1>(a, task, tb, st, c, smem) : eng_attn_t<2, 2>(a, task, tb, st, c, smem);
    fail_dev(c, QTTS_EDEVICE);
    return task;
}

// Combine the splits of one (row, query head): flash-decode merge.  Thread
// (dim d, quarter q) loads dim d of splits q, q + 4, ... of the first 32
// while threads 0.. also load every split's (max, sum): one round trip for
// up to 32 splits, one more per further 32 (long caches).  The quarters'
// weighted sums are added in quarter order (a fixed order: the result does
// not depend on timing).
template <class CT>
__device__ __forceinline__ int eng_combine(const KCONST EngCombine &cb, int task, uint32_t tb, CT &c, float *smem) {
    // Splits are read in rounds of kCombRound; thread (q, d) holds dim d of
    // splits r0 + q + NQ i of a round, and adds them in split order.
    constexpr int HD = 128, NQ = kEngThreads / HD, kCombRound = 32, NS = kCombRound / NQ;
    static_assert(kEngThreads % HD == 0 && kCombRound % NQ == 0 && kEngMaxSplit % kCombRound == 0 &&
                      kEngMaxSplit <= kEngThreads,
                  "combine layout");
    const int m = task / cb.nq, h = task - m * cb.nq;
    const int tid = threadIdx.x, d = tid % HD, q = tid / HD;
    const int ns = cb.nsplit;
    const tv_t *base = cb.part + ((size_t)m * cb.nq + h) * ns * (HD + 2);
    float *sm = smem;                   // [kEngMaxSplit] split max
    float *sl = smem + kEngMaxSplit;    // [kEngMaxSplit] split sum
    float *po = sl + kEngMaxSplit;      // [NQ][HD] weighted P.V sums of each quarter
    float *pl = po + NQ * HD;           // [NQ][HD] weighted sums of each quarter
    float os[NS];
    auto round_cnt = [&](int r0) {
        const int n = min(ns - r0, kCombRound);
        return n > q ? (n - q + NQ - 1) / NQ : 0;
    };
    float ml[2];
    if (tid < ns) {
        const tv_t *ptr[2] = {base + (size_t)tid * (HD + 2), base + (size_t)tid * (HD + 2) + 1};
        const uint32_t tg[2] = {tb + cb.part_tag, tb + cb.part_tag};
        wait_list<2>(ptr, tg, 2, ml, c);
    }
    // the first round's partials are polled with the (max, sum) pairs
    wait_strided<NS>(base + (size_t)q * (HD + 2) + 2 + d, (size_t)NQ * (HD + 2), round_cnt(0), tb + cb.part_tag, os,
                     c);
    if (tid < ns) {
        sm[tid] = ml[0];
        sl[tid] = ml[1];
    }
    __syncthreads();
    float mx = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < kCombRound; sp++)
        if (sp < ns) mx = fmaxf(mx, sm[sp]);
    for (int sp = kCombRound; sp < ns; sp++) mx = fmaxf(mx, sm[sp]);
    float o = 0.0f, l = 0.0f;
    const int cnt = round_cnt(0);
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const int sp = q + NQ * i;
        if (i >= cnt || sm[sp] == -INFINITY) continue;
        const float w = expf(sm[sp] - mx);
        o += w * os[i];
        l += w * sl[sp];
    }
    for (int r0 = kCombRound; r0 < ns; r0 += kCombRound) {  // caches past 8,192 rows
        const int rc = round_cnt(r0);
        wait_strided<NS>(base + (size_t)(r0 + q) * (HD + 2) + 2 + d, (size_t)NQ * (HD + 2), rc, tb + cb.part_tag, os,
                         c);
#pragma unroll
        for (int i = 0; i < NS; i++) {
            const int sp = r0 + q + NQ * i;
            if (i >= rc || sm[sp] == -INFINITY) continue;
            const float w = expf(sm[sp] - mx);
            o += w * os[i];
            l += w * sl[sp];
        }
    }
    po[q * HD + d] = o;
    pl[q * HD + d] = l;
    __syncthreads();
    if (tid < HD) {
        float ot = 0.0f, lt = 0.0f;
#pragma unroll
        for (int qq = 0; qq < NQ; qq++) {
            ot += po[qq * HD + d];
            lt += pl[qq * HD + d];
        }
        put_tv(&cb.out[(size_t)m * cb.nq * HD + h * HD + d], ot / lt, tb + cb.out_tag);
    }
    return task;
}

// The argmax step: files the code and publishes it as a tagged integer.
template <class CT>
__device__ __forceinline__ void eng_argmax(const KCONST EngArgmax &a, uint32_t tb, const EngState &st, CT &c, uint32_t *codes,
                           int max_codes, float *smem) {
    int anynan = 0;
    const int ix = block_argmax<4096 / kEngThreads>(a.logits, a.n, tb + a.logits_tag, c, smem, &anynan);  // n <= 4096
    if (threadIdx.x == 0) {
        uint32_t code = ix < 0 ? 0u : (uint32_t)ix;
        if (anynan) {
            code = 0u;
            fail_dev(c, QTTS_ENAN);
        }
        if (st.frame < max_codes) st_dev_u32(&codes[(size_t)a.group * max_codes + st.frame], code);
        put_tv_u32(a.code, code, tb + a.code_tag);
    }
    __syncthreads();
}

// First index j with r < p[0] + ... + p[j] (f32, summed in index order), or
// -1; one thread, reads batched like seq_sum.
__device__ __forceinline__ int seq_find(const float *p, int n, float r) {
    float cum = 0.0f;
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        float4 v[8];
#pragma unroll
        for (int q = 0; q < 8; q++) v[q] = *reinterpret_cast<const float4 *>(&p[i + 4 * q]);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            cum += v[q].x;
            if (r < cum) return i + 4 * q;
            cum += v[q].y;
            if (r < cum) return i + 4 * q + 1;
            cum += v[q].z;
            if (r < cum) return i + 4 * q + 2;
            cum += v[q].w;
            if (r < cum) return i + 4 * q + 3;
        }
    }
    for (; i < n; i++) {
        cum += p[i];
        if (r < cum) return i;
    }
    return -1;
}

// Exclusive scan over the block.
__device__ int block_exscan(int v, int *wsum, int *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    __syncthreads();
    if (lane == 63) wsum[wave] = x;
    __syncthreads();
    int base = 0, tot = 0;
    for (int w = 0; w < kEngWaves; w++) {
        if (w < wave) base += wsum[w];
        tot += wsum[w];
    }
    *total = tot;
    __syncthreads();
    return base + x - v;
}

// sample_token (src/generate_new.rs:329-391), same schedule as k_sample:
// the three order-dependent f32 sums on one lane in index order, the rest
// in parallel; the stable top-k by radix select over the float bits.
template <class CT>
__device__ __forceinline__ void eng_sample(const KCONST EngSample &P, uint32_t tb, const EngState &st, EngState *st_out, CT &c,
                           uint32_t *codes, int max_codes, float *smem) {
    const int V = P.vocab, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float *s = smem;
    int *list = reinterpret_cast<int *>(s + V);
    unsigned *hist = reinterpret_cast<unsigned *>(list + V);
    int *wsum = reinterpret_cast<int *>(hist + 256);
    float *fred = reinterpret_cast<float *>(wsum + 8);
    int *ired = reinterpret_cast<int *>(fred + 8);
    int *misc = ired + 8;  // [0] prefix [1] mask [2] remaining [3] nan [4] token [5] count
    float *fmisc = reinterpret_cast<float *>(misc + 8);  // [0] max [1] sum
    uint64_t rng = st.rng;

    {
        constexpr int NS = 4096 / kEngThreads;  // V <= 4096
        float lv[NS];
#pragma unroll
        for (int k = 0; k < NS; k++) {
            const int i = tid + k * kEngThreads;
            lv[k] = i < V ? ld_dev(&P.logits[i]) : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < NS; k++) {
            const int i = tid + k * kEngThreads;
            if (i < V) s[i] = lv[k];
        }
    }
    if (tid == 0) {
        misc[3] = 0;
        misc[4] = 0;
    }
    __syncthreads();
    // prev_tokens = the previous frame's 16 codes (zeros before the first)
    uint32_t *prev = reinterpret_cast<uint32_t *>(misc + 16);
    if (tid < P.num_prev) prev[tid] = st.frame > 0 ? ld_dev_u32(&codes[(size_t)tid * max_codes + st.frame - 1]) : 0u;
    __syncthreads();
    if (tid == 0 && P.penalty != 1.0f) {
        for (int j = 0; j < P.num_prev; j++) {
            const uint32_t t = prev[j];
            if (t < (uint32_t)V) {
                if (s[t] > 0.0f)
                    s[t] /= P.penalty;
                else
                    s[t] *= P.penalty;
            }
        }
    }
    __syncthreads();
    if (P.greedy) {
        float bv = -INFINITY;
        int bi = -1, nan = 0;
        for (int i = tid; i < V; i += kEngThreads) {
            const float v = s[i];
            if (v != v)
                nan = 1;
            else if (bi < 0 || v >= bv) {
                bv = v;
                bi = i;
            }
        }
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
                bv = ov;
                bi = oi;
            }
        }
        const int anynan = __syncthreads_or(nan);
        if (lane == 0) {
            fred[wave] = bv;
            ired[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            float b = -INFINITY;
            int ix = -1;
            for (int w = 0; w < kEngWaves; w++)
                if (ired[w] >= 0 && (ix < 0 || fred[w] > b || (fred[w] == b && ired[w] > ix))) {
                    b = fred[w];
                    ix = ired[w];
                }
            misc[4] = ix < 0 ? 0 : ix;
            misc[3] = anynan;
        }
        __syncthreads();
    } else {
        if (P.temperature != 1.0f)
            for (int i = tid; i < V; i += kEngThreads) s[i] /= P.temperature;
        float mx = -INFINITY;
        for (int i = tid; i < V; i += kEngThreads) mx = fmaxf(mx, s[i]);
        mx = wave_max(mx);
        __syncthreads();
        if (lane == 0) fred[wave] = mx;
        __syncthreads();
        if (tid == 0) {
            float t = -INFINITY;
            for (int w = 0; w < kEngWaves; w++) t = fmaxf(t, fred[w]);
            fmisc[0] = t;
        }
        __syncthreads();
        const float maxv = fmisc[0];
        for (int i = tid; i < V; i += kEngThreads) s[i] = (float)exp((double)(s[i] - maxv));
        __syncthreads();
        if (tid == 0) fmisc[1] = seq_sum(s, V);
        __syncthreads();
        const float sum = fmisc[1];
        for (int i = tid; i < V; i += kEngThreads) s[i] = s[i] / sum;
        __syncthreads();
        if (P.top_k > 0 && P.top_k < V) {
            int nan = 0;
            for (int i = tid; i < V; i += kEngThreads)
                if (s[i] != s[i]) nan = 1;
            const int anynan = __syncthreads_or(nan);
            if (tid == 0) {
                misc[0] = 0;
                misc[1] = 0;
                misc[2] = P.top_k;
                misc[3] = anynan;
            }
            __syncthreads();
            if (!anynan) {
                for (int pass = 0; pass < 4; pass++) {
                    const int shift = 24 - 8 * pass;
                    for (int b = tid; b < 256; b += kEngThreads) hist[b] = 0u;
                    __syncthreads();
                    const unsigned prefix = (unsigned)misc[0], mask = (unsigned)misc[1];
                    for (int i = tid; i < V; i += kEngThreads) {
                        const unsigned key = __float_as_uint(s[i]);
                        if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
                    }
                    __syncthreads();
                    if (wave == 0) {
                        // digits in descending order: lane l holds 255-4l .. 252-4l
                        const int rem = misc[2];
                        int h[4], loc = 0;
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            h[q] = (int)hist[255 - 4 * lane - q];
                            loc += h[q];
                        }
                        int incl = loc;
#pragma unroll
                        for (int off = 1; off < 64; off <<= 1) {
                            const int y = __shfl_up(incl, off, 64);
                            if (lane >= off) incl += y;
                        }
                        const int excl = incl - loc;
                        // the first lane whose range reaches rem holds the digit
                        const bool mine = excl < rem && incl >= rem;
                        if (mine) {
                            int cum = excl, sel = 255 - 4 * lane - 3;
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                if (cum + h[q] >= rem) {
                                    sel = 255 - 4 * lane - q;
                                    break;
                                }
                                cum += h[q];
                            }
                            misc[2] = rem - cum;
                            misc[0] = (int)(prefix | ((unsigned)sel << shift));
                            misc[1] = (int)(mask | (255u << shift));
                        }
                    }
                    __syncthreads();
                }
                const unsigned T = (unsigned)misc[0];
                const int need_eq = misc[2];
                const int per = (V + kEngThreads - 1) / kEngThreads;
                const int i0 = min(V, tid * per), i1 = min(V, i0 + per);
                int neq = 0;
                for (int i = i0; i < i1; i++) neq += (__float_as_uint(s[i]) == T);
                int tot;
                int eq_rank = block_exscan(neq, wsum, &tot);
                int nkeep = 0;
                unsigned keep_bits = 0u;
                for (int i = i0; i < i1; i++) {
                    const unsigned key = __float_as_uint(s[i]);
                    bool keep = key > T;
                    if (key == T) {
                        keep = eq_rank < need_eq;
                        eq_rank++;
                    }
                    if (keep) {
                        keep_bits |= 1u << (i - i0);
                        nkeep++;
                    }
                }
                int pos = block_exscan(nkeep, wsum, &tot);
                for (int i = i0; i < i1; i++)
                    if (keep_bits & (1u << (i - i0))) list[pos++] = i;
                __syncthreads();
                // compact the kept probabilities, in index order, into s[0..tot)
                constexpr int NS = 4096 / kEngThreads;  // V <= 4096
                float kv[NS];
#pragma unroll
                for (int k = 0; k < NS; k++) {
                    const int j = tid + k * kEngThreads;
                    kv[k] = j < tot ? s[list[j]] : 0.0f;
                }
                __syncthreads();
#pragma unroll
                for (int k = 0; k < NS; k++) {
                    const int j = tid + k * kEngThreads;
                    if (j < tot) s[j] = kv[k];
                }
                __syncthreads();
                if (tid == 0) fmisc[1] = seq_sum(s, tot);
                __syncthreads();
                const float sum2 = fmisc[1];
                if (sum2 > 0.0f)
                    for (int j = tid; j < tot; j += kEngThreads) s[j] = s[j] / sum2;
                __syncthreads();
                if (tid == 0) {
                    const float r = simple_rand_dev(&rng);
                    const int j = seq_find(s, tot, r);
                    misc[4] = j < 0 ? 0 : list[j];
                }
            }
            __syncthreads();
        } else {
            if (tid == 0) {
                const float r = simple_rand_dev(&rng);
                const int j = seq_find(s, V, r);
                misc[4] = j < 0 ? 0 : j;
            }
            __syncthreads();
        }
    }
    if (tid == 0) {
        uint32_t tok = (uint32_t)misc[4];
        EngState next = st;
        next.rng = rng;
        if (misc[3]) {
            fail_dev(c, QTTS_ENAN);
        } else if (P.stop_on_eos && tok == P.eos) {
            st_dev_i32(c.done, 1);  // EOS: the rest of this frame is abandoned
        } else {
            if (st.frame < max_codes) st_dev_u32(&codes[st.frame], tok);
            next.pos = st.pos + 1;
            next.kvlen = st.kvlen + 1;
            next.frame = st.frame + 1;
            put_tv_u32(P.tok, tok, tb + P.tok_tag);
        }
        st_dev_i32(&st_out->pos, next.pos);
        st_dev_i32(&st_out->kvlen, next.kvlen);
        st_dev_i32(&st_out->frame, next.frame);
        st_dev_u64(&st_out->rng, next.rng);
    }
    __syncthreads();
}

// Next talker input (src/generate_new.rs:270-286), kEngThreads columns per task.
template <class CT>
__device__ __forceinline__ int eng_embsum(const KCONST EngEmbSum &E, int task, uint32_t tb, const EngState &st, CT &c) {
    const int j = task * kEngThreads + threadIdx.x;
    if (E.mode == 2) {  // publish a plain row (host input) as a tagged vector
        if (j < E.hidden) put_tv(&E.out[j], ld_dev(&E.pad[j]), tb + E.out_tag);
        return task;
    }
    const uint32_t tok = wait_tv_u32(E.tok, tb + E.tok_tag, c);
    if (j >= E.hidden) return task;
    float v = tok < (uint32_t)E.codec_emb.K ? q4_element(E.codec_emb, tok, j) : 0.0f;
    if (E.mode == 0) {
        const tv_t *ptr[kMaxGroups];
        uint32_t tg[kMaxGroups];
        float cv[kMaxGroups];
#pragma unroll
        for (int g = 0; g < kMaxGroups; g++) {
            ptr[g] = g < E.num_groups ? E.code[g] : E.tok;
            tg[g] = tb + (g < E.num_groups ? E.code_tag[g] : E.tok_tag);
        }
        wait_list<kMaxGroups>(ptr, tg, E.num_groups, cv, c);
        float acc = 0.0f;
#pragma unroll
        for (int g = 0; g < kMaxGroups; g++) {
            if (g >= E.num_groups) continue;
            const uint32_t cg = __float_as_uint(cv[g]);
            acc += cg < (uint32_t)E.group_emb[g].K ? q4_element(E.group_emb[g], cg, j) : 0.0f;
        }
        v += acc;
        const float *text = st.frame < E.trailing_len ? E.trailing + (size_t)st.frame * E.hidden : E.pad;
        v += ld_dev(&text[j]);
    }
    put_tv(&E.out[j], v, tb + E.out_tag);
    return task;
}

// Loads one dword of every 64-byte line of an op descriptor when a block
// starts the op.  The compiler re-loads descriptor fields where they are used
// rather than holding them in (spilled) registers; this way the fields the
// epilogue reads after the accumulation hit the scalar cache instead of
// waiting a memory round trip on the critical path.
__device__ __forceinline__ void touch_desc(const KCONST EngOp *op) {
    const KCONST uint32_t *p = reinterpret_cast<const KCONST uint32_t *>(op);
    constexpr int kW = (int)(sizeof(EngOp) / 4);
    uint32_t v[kW / 16 + 2];
#pragma unroll
    for (int i = 0; i < kW / 16 + 1; i++) v[i] = p[i * 16 < kW ? i * 16 : kW - 1];
    v[kW / 16 + 1] = p[kW - 1];
#pragma unroll
    for (int i = 0; i < kW / 16 + 2; i++) asm volatile("" ::"s"(v[i]));
}

}  // namespace

template <bool TR>
__global__ __launch_bounds__(kEngThreads) void k_engine(EngArgs A) {
    __shared__ __align__(16) float smem[kEngSmemFloats];
    __shared__ __align__(16) float kvl[2 * kEngLdsKvPos * 128];  // lds_kv attention: this block's K/V rows
    __shared__ int s_bad;  // set by a thread that saw the abort word or timed out
    if (ld_dev_i32(A.done)) return;
    if (threadIdx.x == 0) s_bad = 0;
    __syncthreads();
    Ctl<TR> c{A.done, A.status, 0u, false, nullptr};
    const int G = gridDim.x;
    for (int f = 0; f < A.ncodes; f++) {
        // Code f: its own tag space, and the state its predecessor's sampler wrote.
        const uint32_t tag_base = A.tag_base + (uint32_t)f * kTagStride;
        const EngState *st_in = A.st + ((A.st0 + f) & 1);
        EngState *st_out = A.st + ((A.st0 + f + 1) & 1);
        c.spins = 0u;
        EngState st;
        st.pos = ld_dev_i32(&st_in->pos);
        st.kvlen = ld_dev_i32(&st_in->kvlen);
        st.frame = ld_dev_i32(&st_in->frame);
        st.pad = 0;
        st.rng = ld_dev_u64(&st_in->rng);
        for (int oi = 0; oi < A.nops; oi++) {
            const KCONST EngOp &op = ((const KCONST EngOp *)A.ops)[oi];
            int t = (int)blockIdx.x - op.rot;  // 0 <= rot < G
            if (t < 0) t += G;
            uint64_t *tr = nullptr;
            if constexpr (TR)
                if (A.trace && t < op.ntasks) tr = A.trace + ((size_t)oi * G + blockIdx.x) * kTraceSlots;
            c.tr = tr;
            if (t < op.ntasks) touch_desc(&op);
            if (TR && tr && threadIdx.x == 0) {
                glb(tr)[0] = wall_clock64();
                glb(tr)[8] = clock64();
            }
            for (; t < op.ntasks; t += G) {
                int fi = -1;  // flag this task sets, if any
                switch (op.kind) {
                    case EOP_GEMV: {
                        // An op of M rows runs as M x its one-row tasks (one
                        // instantiation per panel count keeps the kernel's
                        // registers down); every row's split-K non-owners come
                        // before all owners, so no block waits on a later task.
                        const KCONST EngGemv &g = op.gemv;
                        int row = 0, tt = t;
                        if (g.M > 1) {
                            const int per = g.w.N / (g.epi == EEPI_SWIGLU ? 2 * g.cols : g.cols);  // tasks per K chunk
                            const int non = per * (g.kc - 1);
                            if (t < non * g.M) {
                                row = t / non;
                                tt = t - row * non;
                            } else {
                                const int t2 = t - non * g.M;
                                row = t2 / per;
                                tt = non + (t2 - row * per);
                            }
                        }
                        if (g.epi == EEPI_SWIGLU)
                            fi = eng_gemv_cols<1, 2>(g, tt, tag_base, c, smem, row);
                        else
                            fi = eng_gemv_cols<1, 1>(g, tt, tag_base, c, smem, row);
                        break;
                    }
                    case EOP_ATTN: fi = eng_attn(op.attn, t, tag_base, st, c, smem, kvl); break;
                    case EOP_COMBINE: fi = eng_combine(op.comb, t, tag_base, c, smem); break;
                    case EOP_ARGMAX: eng_argmax(op.amax, tag_base, st, c, A.codes, A.max_codes, smem); break;
                    case EOP_SAMPLE: eng_sample(op.samp, tag_base, st, st_out, c, A.codes, A.max_codes, smem); break;
                    case EOP_EMBSUM: fi = eng_embsum(op.emb, t, tag_base, st, c); break;
                    default: break;
                }
                (void)fi;
                // One barrier between tasks: LDS is reused by the next task, and
                // the block leaves together once any thread has seen an abort.
                if (c.bad) s_bad = 1;
                __syncthreads();
                if (s_bad) return;
            }
            if (TR && tr && threadIdx.x == 0) {
                glb(tr)[1] = wall_clock64();
                glb(tr)[9] = clock64();
            }
        }
        if (f + 1 < A.ncodes) {
            // Code boundary: every value the next code reads from this one (the
            // logits, the last hidden row, the appended K/V rows, the state) was
            // stored device-coherently; once each thread's stores are complete,
            // all blocks arrive, and no block starts the next code before every
            // block has finished this one.  The next code's plain loads (cached
            // K/V rows) touch only lines no block has read in this launch.
            // Block 0 gathers the arrival words and publishes one release word,
            // which the other blocks poll (one word each, not all G).
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            const uint32_t btag = tag_base + kTagStride - 1u;
            if (threadIdx.x == 0) put_tv_u32(A.bar + blockIdx.x, 1u, btag);
            if (blockIdx.x == 0) {
                if (threadIdx.x < 64) {
                    const int lane = (int)threadIdx.x;
                    const int cnt = G > lane ? (G - lane + 63) / 64 : 0;  // <= 4 (G <= 256)
                    float arrived[4];
                    wait_strided<4>(A.bar + lane, 64, cnt, btag, arrived, c);
                    if (lane == 0) put_tv_u32(A.bar + G, 1u, btag);
                }
            } else if (threadIdx.x == 0) {
                (void)wait_tv_u32(A.bar + G, btag, c);
            }
            if (c.bad) s_bad = 1;
            __syncthreads();
            if (s_bad) return;
        }
    }
}

hipError_t launch_engine(hipStream_t st, const EngArgs &a, int grid, bool cooperative) {
    EngArgs args = a;
    void *kargs[] = {&args};
    // the traced kernel only when trace slots are given
    const void *fn = a.trace ? (const void *)k_engine<true> : (const void *)k_engine<false>;
    if (cooperative) return hipLaunchCooperativeKernel(fn, dim3((unsigned)grid), dim3(kEngThreads), kargs, 0, st);
    // The same grid through an ordinary launch: on an otherwise idle device
    // every block of a grid of (CUs x resident blocks per CU) is resident at
    // once; if one were not, the waits on its outputs time out (EDEVICE) and
    // the grid drains.
    return hipLaunchKernel(fn, dim3((unsigned)grid), dim3(kEngThreads), kargs, 0, st);
}

int engine_max_grid() {
    int dev = 0, ncu = 0, per = 0, per_tr = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void *)k_engine<false>, kEngThreads, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_tr, (const void *)k_engine<true>, kEngThreads, 0) != hipSuccess)
        return 0;
    return ncu * (per < 1 || per_tr < 1 ? 0 : 1);
}

}  // namespace qtts
