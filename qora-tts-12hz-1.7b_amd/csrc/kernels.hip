// kernels.hip — gfx950 kernels of the per-code loop.
//
//  k_gemv      Q4 GEMV/GEMM-by-rows over the panel-major layout: 128-bit
//              coalesced weight loads, f32 accumulate, deterministic split-K
//              (partials summed in chunk order by the last block of each
//              output group), with fused prologues (RMSNorm, embedding
//              gather) and epilogues (bias, residual add, SiLU*up, QK-norm +
//              RoPE + KV append, argmax).
//  k_attn      split-K flash-decode GQA attention over the device KV cache.
//  k_sample    sample_token on one workgroup (bit-exact order of sums).
//  k_embed_*   Q4 row dequant gathers and the combined next-step embedding.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <cmath>

#include "../../include/qtts.h"
#include "../../include/qtts_synth.h"
#include "device_common.h"
#include "internal.h"

namespace qtts {

namespace {

// Sum over a 256-thread block; every thread gets the result.
__device__ float block_sum_256(float v, float *scratch /* >= 4 */) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) t += scratch[w];
    return t;
}


}  // namespace

// ---------------------------------------------------------------------------
// Q4 GEMV
// ---------------------------------------------------------------------------
template <int M, int RPT>
__global__ __launch_bounds__(kGemvThreads) void k_gemv(GemvParams P) {
    if (P.d_done && *P.d_done) return;
    __shared__ float red[kMaxM * 4 * 32];
    __shared__ float ybuf[kMaxM * 128];
    __shared__ float scratch[8];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int K = P.w.K, N = P.w.N;
    const int p = blockIdx.x / P.kc;
    const int c = blockIdx.x - p * P.kc;
    const int k0 = c * (kGemvThreads * RPT);

    // 1. input values of this thread's rows, issued first: the loads retire
    //    in order, so the accumulation below can then take each weight row
    //    as it lands instead of waiting for the last one.
    float xv[RPT][M];
    if (P.prologue == PRO_RMSNORM) {
        // rms_norm_f16 (src/gemv.rs:406-417); each wave computes the full
        // sum of squares itself, so no block barrier sits behind the loads.
        float inv[M];
#pragma unroll
        for (int m = 0; m < M; m++) {
            const float *src = P.x + (size_t)(P.norm_src_row0 + m) * P.ldx;
            float ss = 0.0f;
            for (int j = lane * 4; j < K; j += 256) {
                const float4 v = *reinterpret_cast<const float4 *>(src + j);
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
            ss = wave_sum(ss);
            inv[m] = 1.0f / sqrtf(ss / (float)K + 1e-6f);
        }
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const int k = k0 + tid + i * kGemvThreads;
            if (k < K) {
                const float g = f16_to_f32(P.gamma[k]);
#pragma unroll
                for (int m = 0; m < M; m++) {
                    const float v = P.x[(size_t)(P.norm_src_row0 + m) * P.ldx + k] * inv[m] * g;
                    xv[i][m] = v;
                    if (P.norm_out && p == 0) P.norm_out[(size_t)m * P.ldn + k] = v;
                }
            } else {
#pragma unroll
                for (int m = 0; m < M; m++) xv[i][m] = 0.0f;
            }
        }
    } else if (P.prologue == PRO_EMBED) {
        // embed_lookup_q4 (src/gemv.rs:377-400) of row *emb_token.
        const uint32_t tok = *P.emb_token;
        float ev[RPT];
#pragma unroll
        for (int i = 0; i < RPT; i++) ev[i] = 0.0f;
        if (tok < (uint32_t)P.emb.K) q4_gather<RPT>(P.emb, tok, k0 + tid, kGemvThreads, K, ev);
#pragma unroll
        for (int i = 0; i < RPT; i++)
#pragma unroll
            for (int m = 0; m < M; m++) xv[i][m] = ev[i];
    } else {
        // branch-free: a row past K reads row K-1 and is zeroed
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const int k = k0 + tid + i * kGemvThreads;
            const int kc = min(k, K - 1);
#pragma unroll
            for (int m = 0; m < M; m++) xv[i][m] = glb(P.x)[(size_t)m * P.ldx + kc];
#pragma unroll
            for (int m = 0; m < M; m++) xv[i][m] = k < K ? xv[i][m] : 0.0f;
        }
    }

    // 2. weight rows of this chunk: one 128-bit load + one scale per row,
    //    issued back to back with no branch between them.  A thread past the
    //    last row (only in the last chunk) re-reads that row, and its input
    //    is zero; the raw scale bits stay opaque until the accumulation so
    //    that no load result is waited for while the others are issued.
    //    The scales go first and a scheduling barrier keeps the weight rows
    //    after them in issue order, so row i is complete once the loads
    //    issued after it (rows i+1..) are all that is outstanding.
    u32x4 wv[RPT];
    uint32_t sv[RPT];
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const int k = min(k0 + tid + i * kGemvThreads, K - 1);
        sv[i] = __builtin_nontemporal_load(glb(P.w.ws) + (size_t)p * K + k);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const int k = min(k0 + tid + i * kGemvThreads, K - 1);
        wv[i] = __builtin_nontemporal_load(glb(reinterpret_cast<const u32x4 *>(P.w.wq)) + (size_t)p * K + k);
        __builtin_amdgcn_sched_barrier(0);
    }

    // 3. accumulate 32 columns per thread: (scale * x) * nib, minus
    //    8 * sum(scale * x) per column.
    float acc[M][32];
    float sxsum[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        sxsum[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; j++) acc[m][j] = 0.0f;
    }
    // Rows past K (last chunk only) carry a zero input and add nothing.
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        // row i's weights become visible to the compiler only here, so the
        // wait before its FMAs is for row i alone
        asm volatile("" : "+v"(sv[i]), "+v"(wv[i]));
        const float s = f16_to_f32((uint16_t)sv[i]);
        // sa = (scale * x) * 2^24, sb = (scale * x) * 2^20 (exact scalings;
        // the sums carry sum(scale * x) * 2^24)
        float sa[M], sb[M];
#pragma unroll
        for (int m = 0; m < M; m++) {
            sa[m] = s * (xv[i][m] * 16777216.0f);
            sb[m] = sa[m] * 0.0625f;
            sxsum[m] += sa[m];
        }
        const uint32_t wd[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
        q4_mix_row<M, 32>(wd, sa, sb, acc);
    }
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int j = 0; j < 32; j++) acc[m][j] = fmaf(-0x1p-21f, sxsum[m], acc[m][j]);  // -8 * sum(scale * x)

    // 4. block reduction -> this chunk's partial for the panel's 32 columns.
#pragma unroll
    for (int m = 0; m < M; m++) dpp_reduce<32>(acc[m], &red[m * 4 * 32]);
    int gp, group;
    if (P.epilogue == EPI_SWIGLU) {
        const int half = N / 64;
        gp = 2;
        group = p % half;
    } else if (P.epilogue == EPI_QKV) {
        gp = P.head_dim / 32;
        group = p / gp;
    } else {
        gp = 1;
        group = p;
    }
    // A block that alone makes its output group (one K chunk, one panel per
    // group) finishes it from LDS: no partial round trip through memory.
    const bool solo = P.kc == 1 && gp == 1;
    __syncthreads();
    if (tid < M * 32) {
        const int m = tid >> 5, col = tid & 31;
        const float *rw = &red[m * 4 * 32 + col];
        const float s = (rw[0] + rw[32]) + (rw[64] + rw[96]);
        if (solo)
            ybuf[m * 32 + col] = s;
        else
            st_dev(&P.partial[((size_t)c * M + m) * N + p * 32 + col], s);
    }

    // 5. the last block of an output group sums the chunks in order.
    const int gcols = gp * 32;
    if (!solo) {
        wait_stores();
        __syncthreads();
        if (tid == 0) s_last = arrive_dev(&P.counters[group]) == (unsigned)(gp * P.kc - 1);
        __syncthreads();
        if (!s_last) return;
        if (tid == 0) reset_dev(&P.counters[group]);
        for (int idx = tid; idx < M * gcols; idx += kGemvThreads) {
            const int m = idx / gcols, j = idx - m * gcols;
            int col;
            if (P.epilogue == EPI_SWIGLU)
                col = (j < 32) ? group * 32 + j : N / 2 + group * 32 + (j - 32);
            else
                col = group * gcols + j;
            float s = 0.0f;
            for (int cc = 0; cc < P.kc; cc++) s += ld_dev(&P.partial[((size_t)cc * M + m) * N + col]);
            ybuf[m * gcols + j] = s;
        }
    }
    __syncthreads();

    // 6. epilogue
    if (P.epilogue == EPI_STORE) {
        for (int idx = tid; idx < M * 32; idx += kGemvThreads) {
            const int m = idx >> 5, j = idx & 31, col = group * 32 + j;
            float v = ybuf[m * 32 + j];
            if (P.bias) v += P.bias[col];
            if (P.fin == FIN_ARGMAX)
                st_dev(&P.y[(size_t)m * P.ldy + col], v);
            else
                P.y[(size_t)m * P.ldy + col] = v;
        }
    } else if (P.epilogue == EPI_RESID) {
        for (int idx = tid; idx < M * 32; idx += kGemvThreads) {
            const int m = idx >> 5, j = idx & 31, col = group * 32 + j;
            P.y[(size_t)m * P.ldy + col] += ybuf[m * 32 + j];
        }
    } else if (P.epilogue == EPI_SWIGLU) {
        // silu(g) * u, src/talker.rs:342-345, silu = g / (1 + exp(-g)).
        for (int idx = tid; idx < M * 32; idx += kGemvThreads) {
            const int m = idx >> 5, j = idx & 31;
            const float g = ybuf[m * 64 + j], u = ybuf[m * 64 + 32 + j];
            P.y[(size_t)m * P.ldy + group * 32 + j] = (g / (1.0f + expf(-g))) * u;
        }
    } else if (P.epilogue == EPI_QKV) {
        // apply_qk_norm (src/talker.rs:86-99) + split-half RoPE
        // (src/rope.rs:79-92) + KV append (src/talker.rs:299-302).
        const int hd = P.head_dim, half = hd / 2;
        const int head = group;
        const bool is_q = head < P.n_q_heads;
        const bool is_k = !is_q && head < P.n_q_heads + P.n_kv_heads;
        for (int m = 0; m < M; m++) {
            const int pos = (P.d_pos ? *P.d_pos : P.pos_const) + m;
            const int row = (P.d_kvlen ? *P.d_kvlen : P.kvlen_const) + m;
            float *vals = ybuf + m * gcols;
            if (is_q || is_k) {
                const float v = tid < hd ? vals[tid] : 0.0f;
                const float ss = block_sum_256(v * v, scratch);
                const float inv = 1.0f / sqrtf(ss / (float)hd + 1e-6f);
                const uint16_t *gam = is_q ? P.q_norm : P.k_norm;
                float nv = 0.0f;
                if (tid < hd) nv = v * inv * f16_to_f32(gam[tid]);
                __syncthreads();
                if (tid < hd) vals[tid] = nv;
                __syncthreads();
                const bool rotate = !(P.rope_skip_oob && pos >= P.rope_rows);
                if (tid < half) {
                    const float x1 = vals[tid], x2 = vals[tid + half];
                    float o1 = x1, o2 = x2;
                    if (rotate) {
                        const float cs = P.rope_cos[(size_t)pos * half + tid];
                        const float sn = P.rope_sin[(size_t)pos * half + tid];
                        o1 = x1 * cs - x2 * sn;
                        o2 = x2 * cs + x1 * sn;
                    }
                    if (is_q) {
                        P.y[(size_t)m * P.ldy + head * hd + tid] = o1;
                        P.y[(size_t)m * P.ldy + head * hd + tid + half] = o2;
                    } else {
                        const int kh = head - P.n_q_heads;
                        float *dst = P.kcache + ((size_t)kh * P.kv_cap + row) * hd;
                        dst[tid] = o1;
                        dst[tid + half] = o2;
                    }
                }
                __syncthreads();
            } else {
                const int vh = head - P.n_q_heads - P.n_kv_heads;
                if (tid < hd) P.vcache[((size_t)vh * P.kv_cap + row) * hd + tid] = vals[tid];
            }
        }
    }

    // 7. kernel-wide final step
    if (P.fin == FIN_ARGMAX) {
        const int ngroups = N / 32;
        wait_stores();
        __syncthreads();
        if (tid == 0) s_last = arrive_dev(&P.counters[ngroups]) == (unsigned)(ngroups - 1);
        __syncthreads();
        if (!s_last) return;
        if (tid == 0) reset_dev(&P.counters[ngroups]);
        // sample_argmax (src/code_predictor.rs:328-334): last index of the max.
        float bv = -INFINITY;
        int bi = -1, nan = 0;
        for (int i = tid; i < N; i += kGemvThreads) {
            const float v = ld_dev(&P.y[i]);
            if (v != v)
                nan = 1;
            else if (bi < 0 || v >= bv) {
                bv = v;
                bi = i;
            }
        }
        __shared__ float sv_[kGemvThreads];
        __shared__ int si_[kGemvThreads];
        __shared__ int snan;
        if (tid == 0) snan = 0;
        __syncthreads();
        if (nan) atomicOr(&snan, 1);
        sv_[tid] = bv;
        si_[tid] = bi;
        __syncthreads();
        for (int st = kGemvThreads / 2; st > 0; st >>= 1) {
            if (tid < st) {
                const float ov = sv_[tid + st];
                const int oi = si_[tid + st];
                if (oi >= 0 && (si_[tid] < 0 || ov > sv_[tid] || (ov == sv_[tid] && oi > si_[tid]))) {
                    sv_[tid] = ov;
                    si_[tid] = oi;
                }
            }
            __syncthreads();
        }
        if (tid == 0) {
            if (snan) {
                *P.argmax_out = 0u;
                if (P.status) *P.status = QTTS_ENAN;
            } else {
                *P.argmax_out = (uint32_t)(si_[0] < 0 ? 0 : si_[0]);
            }
        }
    }
}

// The plain single-row GEMV (gemv_q4, src/gemv.rs:263-309): one block of NT
// threads per C-column slice of a 32-column panel, over its whole K (K <= NT *
// RPT).  With C < 32 the S = 32 / C slices of a panel run on blocks 8 apart --
// one XCD, as blocks are dealt to the 8 XCDs round-robin -- so each panel row
// comes from HBM once into that XCD's L2 (the host uses C < 32 only when the
// panels are a multiple of 8).  The input rows go first, then the scales, then
// the weight rows one by one (scheduling barriers keep that issue order), so
// each row's FMAs wait for that row alone while the later rows are still in
// flight.  The column sums are reduced across each wave's lanes by lane swaps
// (lane_reduce32 / lane_reduce16), then across the waves in LDS, where the
// -8 offset is applied once per column from the block's sum of scale * x.
// Same products as k_gemv.
template <int RPT, int NT, int C>
__global__ __launch_bounds__(NT) void k_gemv_plain(DevQ4 w, const float *x, float *y, const float *bias) {
    constexpr int NW = NT / 64, S = 32 / C, DW = q4_slice_dwords<C>();
    __shared__ float red[NW * C];
    __shared__ float sxr[NW];
    const int tid = threadIdx.x, K = w.K;
    const int b = blockIdx.x;
    const int p = S == 1 ? b : (b / (8 * S)) * 8 + (b % 8);  // panel
    const int sl = S == 1 ? 0 : (b % (8 * S)) / 8;           // slice of the panel
    float xv[RPT];
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const int k = tid + i * NT;
        xv[i] = glb(x)[min(k, K - 1)];
        xv[i] = k < K ? xv[i] : 0.0f;
    }
    uint32_t sv[RPT];
    uint32_t wv[RPT][DW];
#pragma unroll
    for (int i = 0; i < RPT; i++) sv[i] = __builtin_nontemporal_load(glb(w.ws) + (size_t)p * K + min(tid + i * NT, K - 1));
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t *wq = reinterpret_cast<const uint8_t *>(w.wq) + sl * (C / 2);
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        q4_slice_load<C>(wq + ((size_t)p * K + min(tid + i * NT, K - 1)) * 16, wv[i]);
        __builtin_amdgcn_sched_barrier(0);
    }
    float acc[1][C];
#pragma unroll
    for (int j = 0; j < C; j++) acc[0][j] = 0.0f;
    float sxsum = 0.0f;
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        asm volatile("" : "+v"(sv[i]));
#pragma unroll
        for (int d = 0; d < DW; d++) asm volatile("" : "+v"(wv[i][d]));
        const float s = f16_to_f32((uint16_t)sv[i]);
        float sa[1], sb[1];
        sa[0] = s * (xv[i] * 16777216.0f);
        sb[0] = sa[0] * 0.0625f;
        sxsum += sa[0];
        q4_mix_row<1, C>(wv[i], sa, sb, acc);
    }
    if constexpr (C == 32)
        lane_reduce32(acc[0], red);
    else if constexpr (C == 16)
        lane_reduce16(acc[0], red);
    else
        dpp_reduce<C>(acc[0], red);
    const float sw = wave_sum(sxsum);
    if ((tid & 63) == 0) sxr[tid >> 6] = sw;
    __syncthreads();
    if (tid < C) {
        // the waves' sums pairwise, in wave order
        float t[NW], u[NW];
#pragma unroll
        for (int i = 0; i < NW; i++) {
            t[i] = red[i * C + tid];
            u[i] = sxr[i];
        }
#pragma unroll
        for (int h = 1; h < NW; h *= 2)
#pragma unroll
            for (int i = 0; i + h < NW; i += 2 * h) {
                t[i] += t[i + h];
                u[i] += u[i + h];
            }
        float v = fmaf(-0x1p-21f, u[0], t[0]);
        const int col = p * 32 + sl * C + tid;
        if (bias) v += bias[col];
        y[col] = v;
    }
}

// Best-effort streaming read (qtts_stream_read_device_ex): a grid of
// `blocks` 256-thread blocks walks the buffer in grid-wide strides, each
// thread keeping U 16-byte loads in flight per step; the words are XORed and
// an empty asm statement takes the result, so the compiler keeps the loads
// (nothing is stored).
template <int U>
__global__ __launch_bounds__(256) void k_stream_read_loop(const u32x4 *p, uint64_t n16) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    unsigned x = 0;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load(glb(p + i + u * stride));
#pragma unroll
        for (int u = 0; u < U; u++) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(glb(p + i));
        x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    asm volatile("" ::"v"(x));
}

// The same with one word per thread and a block per 256 words.
__global__ __launch_bounds__(256) void k_stream_read(const u32x4 *p, uint64_t n16) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n16) return;
    const u32x4 v = __builtin_nontemporal_load(glb(p + i));
    const unsigned x = v.x ^ v.y ^ v.z ^ v.w;
    asm volatile("" ::"v"(x));
}

extern "C" int32_t qtts_stream_read_device_ex(const void *d_buf, uint64_t bytes, int32_t blocks, int32_t unroll,
                                              void *stream) {
    if (!d_buf || bytes == 0 || bytes % 16 != 0 || ((uintptr_t)d_buf & 15) || bytes / 16 > (uint64_t)256 * 0x7FFFFFFF ||
        blocks < 0 || (blocks > 0 && unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8))
        return -1;
    const uint64_t n16 = bytes / 16;
    const hipStream_t st = (hipStream_t)stream;
    const auto *buf = static_cast<const u32x4 *>(d_buf);
    if (blocks == 0) {
        hipLaunchKernelGGL(k_stream_read, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, st, buf, n16);
    } else {
        const dim3 g((unsigned)blocks), t(256);
        switch (unroll) {
            case 1: hipLaunchKernelGGL(k_stream_read_loop<1>, g, t, 0, st, buf, n16); break;
            case 2: hipLaunchKernelGGL(k_stream_read_loop<2>, g, t, 0, st, buf, n16); break;
            case 4: hipLaunchKernelGGL(k_stream_read_loop<4>, g, t, 0, st, buf, n16); break;
            default: hipLaunchKernelGGL(k_stream_read_loop<8>, g, t, 0, st, buf, n16); break;
        }
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// The read floor: one word per thread and a block per 256 words measured as
// fast as every persistent shape (1-8 blocks per CU, 1-8 loads in flight per
// thread) in kernel-trace averages for 4.7, 7.1 and 14.2 MB.
extern "C" int32_t qtts_stream_read_device(const void *d_buf, uint64_t bytes, void *stream) {
    return qtts_stream_read_device_ex(d_buf, bytes, 0, 1, stream);
}

// Scratch of the allocation-free GEMV entry point: split-K partials
// [chunks <= 4][rows <= 4][N <= 16384] f32, then the arrival counters
// [N/32 + 1] (1 MiB + 2.3 KiB).  Each device holds its own copy while the
// library is loaded.  In host code the name is a stand-in, not a device
// address: kernels get the address hipGetSymbolAddress returns.
static __device__ __align__(256) float scratch[kStaticPartialFloats + kStaticCounterWords];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t static_scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device]) return hipSuccess;
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    // the counters must start at zero (every launch leaves them so)
    e = hipMemset(ptr, 0, sizeof(scratch));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) g_scratch_ptr[device] = ptr;
    return e;
}

void *static_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch_ptr[device];
}

// Rows per thread and K chunks of a launch.  Up to 2048 rows a block takes
// its panel's whole K (8 rows per thread at 2048): every weight load of the
// launch is in flight at once and no partial sums go through memory.  Longer
// K is split into chunks of 2048 rows, summed in chunk order.
void plan_gemv(int K, int N, int M, int *kc, int *rpt) {
    (void)N;
    (void)M;
    int r = (K + kGemvThreads - 1) / kGemvThreads;
    r = r <= 1 ? 1 : r <= 2 ? 2 : r <= 4 ? 4 : 8;
    *rpt = r;
    *kc = (K + kGemvThreads * r - 1) / (kGemvThreads * r);
}

template <int M>
static void launch_gemv_m(hipStream_t st, const GemvParams &p) {
    const dim3 grid((unsigned)((p.w.N / 32) * p.kc));
    switch (p.rpt) {
        case 8: hipLaunchKernelGGL((k_gemv<M, 8>), grid, dim3(kGemvThreads), 0, st, p); break;
        case 4: hipLaunchKernelGGL((k_gemv<M, 4>), grid, dim3(kGemvThreads), 0, st, p); break;
        case 2: hipLaunchKernelGGL((k_gemv<M, 2>), grid, dim3(kGemvThreads), 0, st, p); break;
        default: hipLaunchKernelGGL((k_gemv<M, 1>), grid, dim3(kGemvThreads), 0, st, p); break;
    }
}

template <int NT, int C>
static void launch_plain_nc(hipStream_t st, const GemvParams &p, int rpt) {
    const dim3 grid((unsigned)(p.w.N / C)), t(NT);
    switch (rpt) {
        case 1: hipLaunchKernelGGL((k_gemv_plain<1, NT, C>), grid, t, 0, st, p.w, p.x, p.y, p.bias); return;
        case 2: hipLaunchKernelGGL((k_gemv_plain<2, NT, C>), grid, t, 0, st, p.w, p.x, p.y, p.bias); return;
        case 4: hipLaunchKernelGGL((k_gemv_plain<4, NT, C>), grid, t, 0, st, p.w, p.x, p.y, p.bias); return;
        case 6: hipLaunchKernelGGL((k_gemv_plain<6, NT, C>), grid, t, 0, st, p.w, p.x, p.y, p.bias); return;
        default: hipLaunchKernelGGL((k_gemv_plain<8, NT, C>), grid, t, 0, st, p.w, p.x, p.y, p.bias); return;
    }
}

// Block size and slice width of the plain GEMV for a K x N shape, from a
// kernel-trace sweep of (256, 512, 1024 threads) x (32-, 16-, 8-column
// slices) at the config-1 shapes: 256 threads up to K = 2048 (1024 above),
// and 16-column slices when their blocks fill the CUs evenly (or number no
// more than the CUs), else whole panels: 384 half-panel blocks of 2048 ->
// 6144 leave half the CUs with twice the work (4.54 us against 4.39 for 192
// whole panels).  The slices of a panel need the panels in multiples of 8.
// QTTS_GEMV_PLAIN="threads,cols" overrides the choice (a measurement aid).
static int device_cus() {
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] <= 0) {
        int n = 0;
        cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    return cus[dev];
}

static void plain_plan(int K, int N, int *nt, int *c) {
    const bool slices = (N / 32) % 8 == 0;
    const int cus = device_cus(), b16 = N / 16;
    *nt = K <= 2048 ? 256 : 1024;
    *c = slices && (b16 <= cus || b16 % cus == 0) ? 16 : 32;
    static const char *env = std::getenv("QTTS_GEMV_PLAIN");
    if (env) {
        int a = 0, b = 0;
        if (std::sscanf(env, "%d,%d", &a, &b) == 2 && (a == 256 || a == 512 || a == 1024) &&
            (b == 32 || ((b == 16 || b == 8) && slices)) && K <= 8 * a) {
            *nt = a;
            *c = b;
        }
    }
}

static void launch_plain(hipStream_t st, const GemvParams &p) {
    int nt = 256, c = 32;
    plain_plan(p.w.K, p.w.N, &nt, &c);
    int r = (p.w.K + nt - 1) / nt;
    r = r <= 1 ? 1 : r <= 2 ? 2 : r <= 4 ? 4 : r <= 6 ? 6 : 8;
    switch (nt * 100 + c) {
        case 25632: launch_plain_nc<256, 32>(st, p, r); return;
        case 25616: launch_plain_nc<256, 16>(st, p, r); return;
        case 25608: launch_plain_nc<256, 8>(st, p, r); return;
        case 51232: launch_plain_nc<512, 32>(st, p, r); return;
        case 51216: launch_plain_nc<512, 16>(st, p, r); return;
        case 51208: launch_plain_nc<512, 8>(st, p, r); return;
        case 102432: launch_plain_nc<1024, 32>(st, p, r); return;
        case 102416: launch_plain_nc<1024, 16>(st, p, r); return;
        default: launch_plain_nc<1024, 8>(st, p, r); return;
    }
}

void launch_gemv(hipStream_t st, const GemvParams &p) {
    // One row, a plain input and a store, K <= 8192: one block per panel
    // slice over the whole K (no partial sums through memory).
    if (p.M == 1 && p.w.K <= 8 * kGemvWideThreads && p.prologue == PRO_PLAIN && p.epilogue == EPI_STORE &&
        p.fin == FIN_NONE && !p.d_done && (p.kc == 1 || p.w.K > 8 * kGemvThreads)) {
        launch_plain(st, p);
        return;
    }
    switch (p.M) {
        case 1: launch_gemv_m<1>(st, p); break;
        case 2: launch_gemv_m<2>(st, p); break;
        case 3: launch_gemv_m<3>(st, p); break;
        default: launch_gemv_m<4>(st, p); break;
    }
}

// apply_qk_norm (src/talker.rs:86-99) + split-half RoPE (src/rope.rs:79-92)
// + KV append (src/talker.rs:299-302) of one (head, row) per block, with the
// expressions of the GEMV's EPI_QKV epilogue.
__global__ __launch_bounds__(256) void k_qkv_rows(QkvRowsParams P) {
    __shared__ float vals[256];
    __shared__ float scratch[8];
    const int head = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
    const int hd = P.head_dim, half = hd / 2;
    const bool is_q = head < P.n_q_heads;
    const bool is_k = !is_q && head < P.n_q_heads + P.n_kv_heads;
    int pos = P.pos0 + m, row = P.row0 + m;
    float *kcache = P.kcache, *vcache = P.vcache;
    if (P.row_k) {
        pos = P.pos0 + (P.row_pos ? P.row_pos[(size_t)m * P.row_stride] : 0);
        row = P.row0 + (P.row_kv ? P.row_kv[(size_t)m * P.row_stride] : 0);
        kcache = const_cast<float *>(P.row_k[m]) + P.layer_off;
        vcache = const_cast<float *>(P.row_v[m]) + P.layer_off;
    }
    const float *src = P.raw + (size_t)m * P.ldr + (size_t)head * hd;
    if (is_q || is_k) {
        const float v = tid < hd ? src[tid] : 0.0f;
        const float ss = block_sum_256(v * v, scratch);
        const float inv = 1.0f / sqrtf(ss / (float)hd + 1e-6f);
        const uint16_t *gam = is_q ? P.q_norm : P.k_norm;
        if (tid < hd) vals[tid] = v * inv * f16_to_f32(gam[tid]);
        __syncthreads();
        const bool rotate = !(P.rope_skip_oob && pos >= P.rope_rows);
        if (tid < half) {
            const float x1 = vals[tid], x2 = vals[tid + half];
            float o1 = x1, o2 = x2;
            if (rotate) {
                const float cs = P.rope_cos[(size_t)pos * half + tid];
                const float sn = P.rope_sin[(size_t)pos * half + tid];
                o1 = x1 * cs - x2 * sn;
                o2 = x2 * cs + x1 * sn;
            }
            float *dst;
            if (is_q) {
                dst = P.q + (size_t)m * P.ldq + (size_t)head * hd;
            } else {
                const int kh = head - P.n_q_heads;
                dst = kcache + ((size_t)kh * P.kv_cap + row) * hd;
            }
            dst[tid] = o1;
            dst[tid + half] = o2;
        }
    } else {
        const int vh = head - P.n_q_heads - P.n_kv_heads;
        if (tid < hd) vcache[((size_t)vh * P.kv_cap + row) * hd + tid] = src[tid];
    }
}

void launch_qkv_rows(hipStream_t st, const QkvRowsParams &p) {
    hipLaunchKernelGGL(k_qkv_rows, dim3((unsigned)(p.n_q_heads + 2 * p.n_kv_heads), (unsigned)p.M), dim3(256), 0, st,
                       p);
}

// ---------------------------------------------------------------------------
// Attention: one block per (kv head, split, query row).  Both query heads of
// a GQA group share the K/V reads.  Softmax partials (max, sum, unnormalised
// P.V) are combined in split order by the last block of the kv head.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kAttnThreads) void k_attn(AttnParams P) {
    if (P.d_done && *P.d_done) return;
    constexpr int HD = 128;
    constexpr int GMAX = 4;
    __shared__ float qs[GMAX][HD];
    __shared__ float sc[GMAX][kAttnMaxChunk];
    __shared__ __align__(16) float pv[4 * GMAX][HD];  // P.V partials of the 4 waves
    __shared__ float mloc[GMAX], lloc[GMAX];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m = blockIdx.y;
    const int kvh = blockIdx.x / P.nsplit, sp = blockIdx.x - kvh * P.nsplit;
    const int G = P.nq / P.nkv;
    const int L = P.row_k ? P.kvlen_const + (P.row_kv ? P.row_kv[(size_t)m * P.row_stride] : 0) + 1
                          : (P.d_kvlen ? *P.d_kvlen : P.kvlen_const) + m + 1;
    const int chunk = (L + P.nsplit - 1) / P.nsplit;
    const int t0 = sp * chunk;
    const int t1 = min(L, t0 + chunk);
    const int nt = max(0, t1 - t0);

    const float *Kb = (P.row_k ? P.row_k[m] + P.layer_off : P.kcache) + (size_t)kvh * P.kv_cap * HD;
    const float *Vb = (P.row_v ? P.row_v[m] + P.layer_off : P.vcache) + (size_t)kvh * P.kv_cap * HD;
    __shared__ __align__(16) float kn[HD], vn[HD];  // raw mode: the new row's k and v
    const int tnew = P.raw ? L - 1 : -1;            // its position (raw mode)
    if (P.raw) {
        // QK-norm (src/talker.rs:86-99) and split-half RoPE (src/rope.rs:79-92)
        // of this kv head's query heads and, in the split holding the new
        // position, of its k; two heads per round, 128 threads each
        __shared__ float hn[2][HD];
        __shared__ float hs2[4];
        const bool last = nt > 0 && t1 == L;
        const int nh = G + (last ? 1 : 0);
        const int pos = P.pos0 + (P.row_pos ? P.row_pos[(size_t)m * P.row_stride] : 0);
        const bool rotate = !(P.rope_skip_oob && pos >= P.rope_rows);
        const float *rs = P.raw + (size_t)m * P.ldr;
        const int hh0 = tid >> 7, d = tid & (HD - 1);
        // Every global read of this prologue is issued first (one round
        // trip): the raw rows and gammas of each round's two heads, this
        // thread's RoPE pair and the new row's v.
        constexpr int NR = (GMAX + 2) / 2;  // rounds of two heads: G query heads and k
        float vr[NR], gr[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const int hh = 2 * r + hh0;
            const bool isk = hh == G;
            vr[r] = hh < nh ? rs[(size_t)(isk ? P.nq + kvh : kvh * G + hh) * HD + d] : 0.0f;
            gr[r] = hh < nh ? f16_to_f32((isk ? P.k_norm : P.q_norm)[d]) : 0.0f;
        }
        float cs = 1.0f, sn = 0.0f;
        if (rotate && d < HD / 2) {
            cs = P.rope_cos[(size_t)pos * (HD / 2) + d];
            sn = P.rope_sin[(size_t)pos * (HD / 2) + d];
        }
        const float vnew = last && tid < HD ? rs[(size_t)(P.nq + P.nkv + kvh) * HD + tid] : 0.0f;
#pragma unroll
        for (int r = 0; r < NR; r++) {
            if (2 * r >= nh) break;  // uniform
            const int hh = 2 * r + hh0;
            const bool isk = hh == G;
            const float v = vr[r];
            const float w = wave_sum(v * v);
            if (lane == 0) hs2[wave] = w;
            __syncthreads();
            const float inv = 1.0f / sqrtf((hs2[2 * hh0] + hs2[2 * hh0 + 1]) / (float)HD + 1e-6f);
            if (hh < nh) hn[hh0][d] = v * inv * gr[r];
            __syncthreads();
            if (hh < nh && d < HD / 2) {
                const float x1 = hn[hh0][d], x2 = hn[hh0][d + HD / 2];
                float o1 = x1, o2 = x2;
                if (rotate) {
                    o1 = x1 * cs - x2 * sn;
                    o2 = x2 * cs + x1 * sn;
                }
                float *dst = isk ? kn : qs[hh < GMAX ? hh : 0];
                dst[d] = o1;
                dst[d + HD / 2] = o2;
            }
            __syncthreads();
        }
        if (last && tid < HD) {
            // the new row: v as is; k and v appended to the stream's cache
            // (src/talker.rs:299-302) for later steps; this step reads them
            // from LDS
            vn[tid] = vnew;
            const_cast<float *>(Kb)[(size_t)tnew * HD + tid] = kn[tid];
            const_cast<float *>(Vb)[(size_t)tnew * HD + tid] = vn[tid];
        }
    } else {
        for (int idx = tid; idx < G * HD; idx += kAttnThreads) {
            const int g = idx / HD, dd = idx - g * HD;
            qs[g][dd] = P.q[(size_t)m * P.ldq + (size_t)(kvh * G + g) * HD + dd];
        }
    }
    __syncthreads();

    // The first VU * 8 V rows of the split are loaded now, so they are in
    // flight with the K rows (a split of <= 64 positions makes one round
    // trip for K and V together).
    constexpr int VU = 8;
    const int d4 = tid & 31, r8 = tid >> 5;
    float4 v_first[VU];
    if (nt > 0) {
#pragma unroll
        for (int u = 0; u < VU; u++) {
            const int tt = min(r8 + 8 * u, nt - 1);
            v_first[u] = *reinterpret_cast<const float4 *>(Vb + (size_t)(t0 + tt) * HD + 4 * d4);
        }
    }
    // scores: 16 lanes per position, 8 dims per lane; SU positions per
    // thread are loaded before any is used (clamped to the split, masked
    // after), so their loads are in flight together.
    if (nt > 0) {
        constexpr int SU = 4;
        const int l16 = tid & 15, slot = tid >> 4;
        for (int b0 = 0; b0 < nt; b0 += 16 * SU) {
            float4 ka[SU], kb[SU];
#pragma unroll
            for (int u = 0; u < SU; u++) {
                const int tt = min(b0 + slot + 16 * u, nt - 1);
                const float *kr = Kb + (size_t)(t0 + tt) * HD + l16 * 8;
                ka[u] = *reinterpret_cast<const float4 *>(kr);
                kb[u] = *reinterpret_cast<const float4 *>(kr + 4);
            }
#pragma unroll
            for (int u = 0; u < SU; u++) {
                const int tt = min(b0 + slot + 16 * u, nt - 1);
                if (t0 + tt == tnew) {
                    ka[u] = *reinterpret_cast<const float4 *>(&kn[l16 * 8]);
                    kb[u] = *reinterpret_cast<const float4 *>(&kn[l16 * 8 + 4]);
                }
            }
#pragma unroll
            for (int u = 0; u < SU; u++) {
                const int tt = b0 + slot + 16 * u;
                for (int g = 0; g < G; g++) {
                    const float *qq = &qs[g][l16 * 8];
                    float dot = qq[0] * ka[u].x + qq[1] * ka[u].y + qq[2] * ka[u].z + qq[3] * ka[u].w +
                                qq[4] * kb[u].x + qq[5] * kb[u].y + qq[6] * kb[u].z + qq[7] * kb[u].w;
                    dot += __shfl_xor(dot, 8, 16);
                    dot += __shfl_xor(dot, 4, 16);
                    dot += __shfl_xor(dot, 2, 16);
                    dot += __shfl_xor(dot, 1, 16);
                    if (l16 == 0 && tt < nt) sc[g][tt] = dot * P.scale;
                }
            }
        }
    }
    __syncthreads();
    // local softmax statistics, one wave per query head.
    for (int g = wave; g < G; g += kAttnThreads / 64) {
        float mx = -INFINITY;
        for (int t = lane; t < nt; t += 64) mx = fmaxf(mx, sc[g][t]);
        mx = wave_max(mx);
        float l = 0.0f;
        for (int t = lane; t < nt; t += 64) {
            const float e = expf(sc[g][t] - mx);
            sc[g][t] = e;
            l += e;
        }
        l = wave_sum(l);
        if (lane == 0) {
            mloc[g] = nt > 0 ? mx : -INFINITY;
            lloc[g] = l;
        }
    }
    __syncthreads();
    // P.V: thread (d4, r8) holds dims 4*d4..4*d4+3 of every 8th position
    // from r8, VU rows loaded together (the first VU above); the two halves
    // of a wave are added by a lane exchange and the 4 waves through LDS.
    {
        float4 acc[GMAX];
#pragma unroll
        for (int g = 0; g < GMAX; g++) acc[g] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int b0 = 0; b0 < nt; b0 += 8 * VU) {
            float4 v[VU];
#pragma unroll
            for (int u = 0; u < VU; u++) {
                const int tt = min(b0 + r8 + 8 * u, nt - 1);
                v[u] = b0 == 0 ? v_first[u] : *reinterpret_cast<const float4 *>(Vb + (size_t)(t0 + tt) * HD + 4 * d4);
            }
#pragma unroll
            for (int u = 0; u < VU; u++) {
                const int tt = min(b0 + r8 + 8 * u, nt - 1);
                if (t0 + tt == tnew) v[u] = *reinterpret_cast<const float4 *>(&vn[4 * d4]);
            }
#pragma unroll
            for (int u = 0; u < VU; u++) {
                const int tt = b0 + r8 + 8 * u;
                if (tt >= nt) continue;
#pragma unroll
                for (int g = 0; g < GMAX; g++) {
                    if (g >= G) continue;
                    const float pr = sc[g][tt];
                    acc[g].x += pr * v[u].x;
                    acc[g].y += pr * v[u].y;
                    acc[g].z += pr * v[u].z;
                    acc[g].w += pr * v[u].w;
                }
            }
        }
        float *red = &pv[0][0];  // [4 waves][GMAX][HD]
#pragma unroll
        for (int g = 0; g < GMAX; g++) {
            acc[g].x += __shfl_xor(acc[g].x, 32);
            acc[g].y += __shfl_xor(acc[g].y, 32);
            acc[g].z += __shfl_xor(acc[g].z, 32);
            acc[g].w += __shfl_xor(acc[g].w, 32);
            if (lane < 32 && g < G)
                *reinterpret_cast<float4 *>(&red[(wave * GMAX + g) * HD + 4 * d4]) = acc[g];
        }
        __syncthreads();
        for (int idx = tid; idx < G * HD; idx += kAttnThreads) {
            const int g = idx / HD, d = idx - g * HD;
            const float o = (red[g * HD + d] + red[(GMAX + g) * HD + d]) +
                            (red[(2 * GMAX + g) * HD + d] + red[(3 * GMAX + g) * HD + d]);
            const int h = kvh * G + g;
            if (P.nsplit == 1) {
                // one split: the combine below would give (1 * o) / (1 * l)
                P.out[(size_t)m * P.ldo + (size_t)h * HD + d] = o / lloc[g];
            } else {
                float *dst = P.part + (((size_t)m * P.nq + h) * P.nsplit + sp) * (HD + 2);
                st_dev(&dst[2 + d], o);
                if (d == 0) {
                    st_dev(&dst[0], mloc[g]);
                    st_dev(&dst[1], lloc[g]);
                }
            }
        }
    }
    if (P.nsplit == 1) return;
    wait_stores();
    __syncthreads();
    if (tid == 0) s_last = arrive_dev(&P.counters[m * P.nkv + kvh]) == (unsigned)(P.nsplit - 1);
    __syncthreads();
    if (!s_last) return;
    if (tid == 0) reset_dev(&P.counters[m * P.nkv + kvh]);
    // Combine the splits (flash-decode merge, in split order).  The splits'
    // (max, sum) pairs are staged in LDS and each thread's P.V partials are
    // read CB at a time, so the device-coherent loads overlap.
    const int ns = P.nsplit;
    const bool staged = G * ns <= GMAX * kAttnMaxChunk / 2;
    float *sm = &sc[0][0], *sl = sm + GMAX * kAttnMaxChunk / 2;  // [G][ns] each
    if (staged) {
        for (int i = tid; i < G * ns; i += kAttnThreads) {
            const int g = i / ns, s2 = i - g * ns;
            const float *src = P.part + (((size_t)m * P.nq + kvh * G + g) * ns + s2) * (HD + 2);
            sm[i] = ld_dev(&src[0]);
            sl[i] = ld_dev(&src[1]);
        }
    }
    __syncthreads();
    for (int idx = tid; idx < G * HD; idx += kAttnThreads) {
        const int g = idx / HD, d = idx - g * HD;
        const int h = kvh * G + g;
        const float *base = P.part + ((size_t)m * P.nq + h) * ns * (HD + 2);
        auto mval = [&](int s2) { return staged ? sm[g * ns + s2] : ld_dev(&base[s2 * (HD + 2)]); };
        auto lval = [&](int s2) { return staged ? sl[g * ns + s2] : ld_dev(&base[s2 * (HD + 2) + 1]); };
        float mx = -INFINITY;
        for (int s2 = 0; s2 < ns; s2++) mx = fmaxf(mx, mval(s2));
        float o = 0.0f, l = 0.0f;
        constexpr int CB = 32;
        for (int s0 = 0; s0 < ns; s0 += CB) {
            float ov[CB];
#pragma unroll
            for (int u = 0; u < CB; u++) ov[u] = s0 + u < ns ? ld_dev(&base[(s0 + u) * (HD + 2) + 2 + d]) : 0.0f;
#pragma unroll
            for (int u = 0; u < CB; u++) {
                if (s0 + u >= ns) continue;
                const float ms = mval(s0 + u);
                if (ms == -INFINITY) continue;
                const float w = expf(ms - mx);
                o += w * ov[u];
                l += w * lval(s0 + u);
            }
        }
        P.out[(size_t)m * P.ldo + (size_t)h * HD + d] = o / l;
    }
}

void launch_attention(hipStream_t st, const AttnParams &p, int M) {
    hipLaunchKernelGGL(k_attn, dim3((unsigned)(p.nkv * p.nsplit), (unsigned)M), dim3(kAttnThreads), 0, st, p);
}

// ---------------------------------------------------------------------------
// Sampler: sample_token (src/generate_new.rs:329-391) on one workgroup.  The
// three order-dependent f32 sums (softmax denominator, top-k renormaliser,
// cumulative sum) run sequentially in index order on one lane, as in the
// reference; everything else is order-independent and runs in parallel.
// exp is evaluated in double and rounded once to float (glibc's expf is
// accurate to 0.502 ulp, so both agree except within ~0.002 ulp of a
// rounding boundary).
// ---------------------------------------------------------------------------
namespace {

// Exclusive scan over a 1024-thread block.
__device__ int block_exscan_1024(int v, int *wsum /* >= 16 */, int *total) {
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
    for (int w = 0; w < (int)(blockDim.x >> 6); w++) {
        if (w < wave) base += wsum[w];
        tot += wsum[w];
    }
    *total = tot;
    return base + x - v;
}

}  // namespace

template <class T>
__device__ __forceinline__ T *byte_off(T *p, long long bytes) {
    return p ? reinterpret_cast<T *>(reinterpret_cast<char *>(const_cast<typename std::remove_const<T>::type *>(p)) +
                                     bytes)
             : p;
}

__global__ __launch_bounds__(kSampleThreads) void k_sample(SampleParams Pin) {
    SampleParams P = Pin;
    if (Pin.batch > 1) {
        const long long b = blockIdx.x, so = b * Pin.state_stride;
        P.logits += b * Pin.logits_stride;
        P.prev = byte_off(P.prev, so);
        P.rng = byte_off(P.rng, so);
        P.token_out = byte_off(P.token_out, so);
        P.status = byte_off(P.status, so);
        P.done = byte_off(P.done, so);
        P.frame = byte_off(P.frame, so);
        P.prev_out = byte_off(P.prev_out, so);
        if (P.codes) P.codes += b * Pin.codes_stride;
    }
    if (P.done && *P.done) return;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    float *s = reinterpret_cast<float *>(smem_raw);
    int *list = reinterpret_cast<int *>(s + P.vocab);
    __shared__ unsigned hist[256];
    __shared__ int wsum[16];
    __shared__ float fred[16];
    __shared__ int ired[16];
    __shared__ float s_max, s_sum;
    __shared__ unsigned s_prefix, s_mask;
    __shared__ int s_remaining, s_nan, s_count;
    __shared__ uint32_t s_token;
    __shared__ uint32_t s_prev[32];  // n_prev <= 32

    const int V = P.vocab, tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & 63, wave = tid >> 6, nwaves = nthr >> 6;
    for (int i = tid; i < V; i += nthr) s[i] = P.logits[i];
    if (tid < P.n_prev) s_prev[tid] = P.prev[tid];  // loaded with the logits, not one by one below
    if (tid == 0) {
        s_nan = 0;
        s_token = 0;
    }
    __syncthreads();
    if (tid == 0 && P.penalty != 1.0f) {
        for (int j = 0; j < P.n_prev; j++) {
            const uint32_t t = s_prev[j];
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
        // argmax with the last index winning ties (src/generate.rs:51-56).
        float bv = -INFINITY;
        int bi = -1, nan = 0;
        for (int i = tid; i < V; i += nthr) {
            const float v = s[i];
            if (v != v)
                nan = 1;
            else if (bi < 0 || v >= bv) {
                bv = v;
                bi = i;
            }
        }
        if (nan) atomicOr(&s_nan, 1);
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(bv, off, 64);
            const int oi = __shfl_xor(bi, off, 64);
            if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi > bi))) {
                bv = ov;
                bi = oi;
            }
        }
        if (lane == 0) {
            fred[wave] = bv;
            ired[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            float b = -INFINITY;
            int ix = -1;
            for (int w = 0; w < nwaves; w++) {
                if (ired[w] >= 0 && (ix < 0 || fred[w] > b || (fred[w] == b && ired[w] > ix))) {
                    b = fred[w];
                    ix = ired[w];
                }
            }
            s_token = ix < 0 ? 0u : (uint32_t)ix;
        }
        __syncthreads();
    } else {
        if (P.temperature != 1.0f)
            for (int i = tid; i < V; i += nthr) s[i] /= P.temperature;
        // max (fold with f32::max: NaN is ignored)
        float mx = -INFINITY;
        for (int i = tid; i < V; i += nthr) mx = fmaxf(mx, s[i]);
        mx = wave_max(mx);
        if (lane == 0) fred[wave] = mx;
        __syncthreads();
        if (tid == 0) {
            float t = -INFINITY;
            for (int w = 0; w < nwaves; w++) t = fmaxf(t, fred[w]);
            s_max = t;
        }
        __syncthreads();
        const float maxv = s_max;
        for (int i = tid; i < V; i += nthr) s[i] = (float)exp((double)(s[i] - maxv));
        __syncthreads();
        if (tid == 0) s_sum = seq_sum(s, V);
        __syncthreads();
        const float sum = s_sum;
        for (int i = tid; i < V; i += nthr) s[i] = s[i] / sum;
        __syncthreads();

        const bool topk = P.top_k > 0 && P.top_k < V;
        if (topk) {
            // The stable descending sort keeps entry i iff
            //   #{j: s_j > s_i} + #{j < i: s_j == s_i} < top_k.
            // Find the top_k-th largest key by MSB-first radix select over
            // the float bits (all values are >= 0, so bits order as values).
            int nan = 0;
            for (int i = tid; i < V; i += nthr)
                if (s[i] != s[i]) nan = 1;
            if (nan) atomicOr(&s_nan, 1);
            if (tid == 0) {
                s_prefix = 0u;
                s_mask = 0u;
                s_remaining = P.top_k;
            }
            __syncthreads();
            if (!s_nan) {
                for (int pass = 0; pass < 4; pass++) {
                    const int shift = 24 - 8 * pass;
                    for (int b = tid; b < 256; b += nthr) hist[b] = 0u;
                    __syncthreads();
                    const unsigned prefix = s_prefix, mask = s_mask;
                    for (int i = tid; i < V; i += nthr) {
                        const unsigned key = __float_as_uint(s[i]);
                        if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
                    }
                    __syncthreads();
                    if (wave == 0) {
                        // the digit holding the rem-th largest key, as a wave
                        // scan: lane l holds digits 255-4l .. 252-4l
                        const int rem = s_remaining;
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
                        if (excl < rem && incl >= rem) {  // one lane: the count with the prefix is >= rem
                            int cum = excl, sel = 255 - 4 * lane - 3;
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                if (cum + h[q] >= rem) {
                                    sel = 255 - 4 * lane - q;
                                    break;
                                }
                                cum += h[q];
                            }
                            s_remaining = rem - cum;
                            s_prefix = prefix | ((unsigned)sel << shift);
                            s_mask = mask | (255u << shift);
                        }
                    }
                    __syncthreads();
                }
                const unsigned T = s_prefix;
                const int need_eq = s_remaining;
                // contiguous ownership keeps index order for the scans
                const int per = (V + nthr - 1) / nthr;
                const int i0 = min(V, tid * per), i1 = min(V, i0 + per);
                int neq = 0;
                for (int i = i0; i < i1; i++) neq += (__float_as_uint(s[i]) == T);
                int tot;
                int eq_rank = block_exscan_1024(neq, wsum, &tot);
                int nkeep = 0;
                unsigned keep_bits = 0u;  // per <= 32
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
                __syncthreads();
                int pos = block_exscan_1024(nkeep, wsum, &tot);
                for (int i = i0; i < i1; i++)
                    if (keep_bits & (1u << (i - i0))) list[pos++] = i;
                if (tid == 0) s_count = tot;
                __syncthreads();
                if (tid == 0) {
                    const int cnt = s_count;
                    float sum2 = 0.0f;
                    for (int j = 0; j < cnt; j++) sum2 += s[list[j]];
                    const float r = simple_rand_dev(P.rng);
                    float cumsum = 0.0f;
                    uint32_t tok = 0u;
                    for (int j = 0; j < cnt; j++) {
                        const float pj = sum2 > 0.0f ? s[list[j]] / sum2 : s[list[j]];
                        cumsum += pj;
                        if (r < cumsum) {
                            tok = (uint32_t)list[j];
                            break;
                        }
                    }
                    s_token = tok;
                }
            }
            __syncthreads();
        } else {
            if (tid == 0) {
                const float r = simple_rand_dev(P.rng);
                float cumsum = 0.0f;
                uint32_t tok = 0u;
                for (int i = 0; i < V; i++) {
                    cumsum += s[i];
                    if (r < cumsum) {
                        tok = (uint32_t)i;
                        break;
                    }
                }
                s_token = tok;
            }
            __syncthreads();
        }
    }

    if (tid == 0) {
        uint32_t tok = s_token;
        if (s_nan) {
            tok = 0u;
            if (P.status) *P.status = QTTS_ENAN;
            if (P.done) *P.done = 1;
        } else if (P.done && P.stop_on_eos && tok == P.eos) {
            *P.done = 1;
        } else {
            if (P.codes && P.frame) {
                const int f = *P.frame;
                if (f < P.max_codes) P.codes[f] = tok;
            }
            if (P.prev_out) P.prev_out[0] = tok;
        }
        *P.token_out = tok;
    }
}

void launch_sample(hipStream_t st, const SampleParams &p) {
    const size_t smem = (size_t)p.vocab * (sizeof(float) + sizeof(int));
    hipLaunchKernelGGL(k_sample, dim3((unsigned)(p.batch > 1 ? p.batch : 1)), dim3(kSampleThreads), smem, st, p);
}

// ---------------------------------------------------------------------------
// Embedding gathers
// ---------------------------------------------------------------------------
__global__ void k_embed_row(DevQ4 w, const uint32_t *tok, float *out, const int *d_done) {
    if (d_done && *d_done) return;
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= w.N) return;
    const uint32_t t = *tok;
    out[j] = t < (uint32_t)w.K ? q4_element(w, t, j) : 0.0f;
}

void launch_embed_row(hipStream_t st, const DevQ4 &w, const uint32_t *d_token, float *out, const int *d_done) {
    hipLaunchKernelGGL(k_embed_row, dim3((unsigned)((w.N + 255) / 256)), dim3(256), 0, st, w, d_token, out, d_done);
}

// Next talker input: codec_emb[code0] + sum_g group_emb[g][code_g] + text row
// (src/generate_new.rs:270-286, src/code_predictor.rs:280-293), in the
// reference's order of additions; the frame's codes are filed here too.
__global__ void k_embed_sum(EmbSumParams Pin) {
    EmbSumParams P = Pin;
    if (Pin.batch > 1) {
        const long long b = blockIdx.y, so = b * Pin.state_stride;
        P.cur = byte_off(P.cur, so);
        P.frame = byte_off(P.frame, so);
        P.d_done = byte_off(P.d_done, so);
        P.prev = byte_off(P.prev, so);
        if (P.trailing) P.trailing += b * Pin.trailing_stride;
        P.out += b * Pin.out_stride;
        if (P.codes) P.codes += b * Pin.codes_stride;
    }
    if (P.d_done && *P.d_done) return;
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    const int frame = P.frame ? *P.frame : 0;
    if (blockIdx.x == 0 && threadIdx.x < (unsigned)P.num_groups) {
        const int g = threadIdx.x;
        if (P.codes && frame < P.max_codes) P.codes[(size_t)(g + 1) * P.max_codes + frame] = P.cur[1 + g];
        if (P.prev) P.prev[1 + g] = P.cur[1 + g];
    }
    if (j >= P.hidden) return;
    // Every code, then every element's byte and scale, are loaded before any
    // is used (two memory round trips instead of two per group).  Slot 0 is
    // code 0's codec_emb row (mode 0), slot 1 + g group g's row; a slot past
    // the groups reads row 0 of a table this mode has (codec_emb in mode 0,
    // group 0's in mode 1) and is not used.
    constexpr int NG = kMaxGroups + 1;
    const bool full = P.mode != 1;
    const int ng = P.num_groups;
    if (!full && ng <= 0) {  // an empty acoustic sum
        P.out[j] = 0.0f;
        return;
    }
    const bool text_in = full && ng > 0;
    float text = 0.0f;
    if (text_in) text = (frame < P.trailing_len ? P.trailing + (size_t)frame * P.hidden : P.pad)[j];
    uint32_t code[NG];
#pragma unroll
    for (int g = 0; g < NG; g++) code[g] = g <= ng ? P.cur[g] : 0u;
    uint32_t by[NG], sc[NG];
    bool ok[NG];
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const bool used = g == 0 ? full : g - 1 < ng;
        const DevQ4 &w = g > 0 && g - 1 < ng ? P.group_emb[g - 1] : (full ? P.codec_emb : P.group_emb[0]);
        ok[g] = used && code[g] < (uint32_t)w.K;
        const size_t r = (size_t)(j >> 5) * w.K + (ok[g] ? code[g] : 0u);
        by[g] = glb(reinterpret_cast<const uint8_t *>(w.wq))[r * 16 + ((j & 31) >> 1)];
        sc[g] = glb(w.ws)[r];
    }
#pragma unroll
    for (int g = 0; g < NG; g++) asm volatile("" : "+v"(by[g]), "+v"(sc[g]));
    // embed_lookup_q4 elements (src/gemv.rs:388-396), summed in the order of
    // src/code_predictor.rs:280-293 and src/generate_new.rs:270-286
    const auto elem = [&](int g) {
        const int nib = (j & 1) ? (int)(by[g] >> 4) : (int)(by[g] & 15u);
        return ok[g] ? f16_to_f32((uint16_t)sc[g]) * (float)(nib - 8) : 0.0f;
    };
    float acc = 0.0f;
#pragma unroll
    for (int g = 1; g < NG; g++)
        if (g - 1 < ng) acc += elem(g);
    if (!full) {  // get_acoustic_embeddings_sum alone
        P.out[j] = acc;
        return;
    }
    float v = elem(0);
    if (ng > 0) {
        v += acc;
        v += text;
    }
    P.out[j] = v;
}

void launch_embed_sum(hipStream_t st, const EmbSumParams &p) {
    hipLaunchKernelGGL(k_embed_sum, dim3((unsigned)((p.hidden + 255) / 256), (unsigned)(p.batch > 1 ? p.batch : 1)),
                       dim3(256), 0, st, p);
}

__global__ void k_advance(LoopState *states, int frame_step, int batch) {
    const int b = threadIdx.x;
    if (b >= batch) return;
    LoopState *s = states + b;
    if (s->done) return;
    s->pos += 1;
    s->kvlen += 1;
    s->frame += frame_step;
}

void launch_advance(hipStream_t st, LoopState *s, int frame_step, int batch) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3((unsigned)((batch + 63) / 64 * 64)), 0, st, s, frame_step, batch);
}

// The prompt rows of prefill_custom_voice (src/generate_new.rs:84-177): a
// codec embedding row plus a text-projection row, added element by element
// in that order, or one row copied as it is.
__global__ void k_prompt_rows(PromptRowsParams P) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
    if (j >= P.H || r >= P.L) return;
    const float v = P.a[r][j];
    P.out[(size_t)r * P.H + j] = P.b[r] ? v + P.b[r][j] : v;
}

void launch_prompt_rows(hipStream_t st, const PromptRowsParams &p) {
    hipLaunchKernelGGL(k_prompt_rows, dim3((unsigned)((p.H + 255) / 256), (unsigned)p.L), dim3(256), 0, st, p);
}

// silu between the two text-projection layers (src/talker.rs:111-112).
__global__ void k_silu(float *x, long long n) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    x[i] = v / (1.0f + expf(-v));
}

void launch_silu(hipStream_t st, float *x, long long n) {
    hipLaunchKernelGGL(k_silu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n);
}

// generate::sample_top_k (src/generate.rs:50-84), the legacy sampler:
//  - temperature <= 0: greedy, the last of equal maxima (Iterator::max_by);
//  - else the top_k largest logits in descending order (the reference's
//    sort_unstable_by leaves equal logits in an unspecified order; here they
//    go by ascending index), p_i = exp((l_i - l_0) / T) summed in that
//    order, each divided by the sum, then the first i in that order with
//    r < cumsum, else the k-th index.
// A NaN logit (partial_cmp().unwrap() panics) sets *status = QTTS_ENAN.  The
// sort is a bitonic sort of (logit, index) pairs in LDS; the sums run on one
// thread in the reference's order.
__global__ __launch_bounds__(1024) void k_sample_top_k(TopKParams P) {
    __shared__ float key[kTopKMaxVocab];
    __shared__ int idx[kTopKMaxVocab];
    __shared__ int s_nan;
    const int tid = threadIdx.x, V = P.vocab;
    int n2 = 1;
    while (n2 < V) n2 <<= 1;
    if (tid == 0) s_nan = 0;
    __syncthreads();
    int nan = 0;
    for (int i = tid; i < n2; i += blockDim.x) {
        const float v = i < V ? P.logits[i] : -INFINITY;
        if (v != v) nan = 1;
        key[i] = v;
        idx[i] = i < V ? i : 0x7fffffff;
    }
    if (nan) atomicOr(&s_nan, 1);
    __syncthreads();
    if (s_nan) {
        if (tid == 0) {
            *P.status = QTTS_ENAN;
            *P.token_out = 0u;
        }
        return;
    }
    if (P.temperature <= 0.0f) {
        // the last index of the maximum: thread 0 scans in index order
        if (tid == 0) {
            int best = 0;
            for (int i = 1; i < V; i++)
                if (key[i] >= key[best]) best = i;
            *P.token_out = (uint32_t)best;
            *P.status = 0;
        }
        return;
    }
    // bitonic sort, descending by logit, ascending index among equals
    for (int size = 2; size <= n2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < n2; i += blockDim.x) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool desc = (i & size) == 0;
                    const float ki = key[i], kj = key[j];
                    const int ii = idx[i], ij = idx[j];
                    const bool i_first = ki > kj || (ki == kj && ii < ij);
                    if (desc != i_first) {
                        key[i] = kj;
                        key[j] = ki;
                        idx[i] = ij;
                        idx[j] = ii;
                    }
                }
            }
            __syncthreads();
        }
    }
    if (tid == 0) {
        const int k = P.top_k < V ? P.top_k : V;
        const float maxv = key[0];
        float sum = 0.0f;
        for (int i = 0; i < k; i++) {
            const float p = (float)exp((double)((key[i] - maxv) / P.temperature));
            key[i] = p;
            sum += p;
        }
        for (int i = 0; i < k; i++) key[i] /= sum;
        uint64_t st = *P.rng;
        const float r = simple_rand_dev(&st);
        *P.rng = st;
        uint32_t tok = (uint32_t)idx[k - 1];
        float cumsum = 0.0f;
        for (int i = 0; i < k; i++) {
            cumsum += key[i];
            if (r < cumsum) {
                tok = (uint32_t)idx[i];
                break;
            }
        }
        *P.token_out = tok;
        *P.status = 0;
    }
}

void launch_sample_top_k(hipStream_t st, const TopKParams &p) {
    hipLaunchKernelGGL(k_sample_top_k, dim3(1), dim3(1024), 0, st, p);
}

// Row r = embedding row tok[r * tok_stride] of w (embed_lookup_q4,
// src/gemv.rs:377-400, exact), at out + r * out_stride.
__global__ void k_embed_rows(DevQ4 w, const uint32_t *tok, long long tok_stride, float *out, long long out_stride) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
    if (j >= w.N) return;
    const uint32_t t = tok[(size_t)r * tok_stride];
    out[(size_t)r * out_stride + j] = t < (uint32_t)w.K ? q4_element(w, t, j) : 0.0f;
}

void launch_embed_rows(hipStream_t st, const DevQ4 &w, const uint32_t *tok, long long tok_stride, int rows, float *out,
                       long long out_stride) {
    hipLaunchKernelGGL(k_embed_rows, dim3((unsigned)((w.N + 255) / 256), (unsigned)rows), dim3(256), 0, st, w, tok,
                       tok_stride, out, out_stride);
}

// The rows of prefill_talker (src/talker.rs:475-484): row r is text row
// slot[r] (already projected) when slot[r] >= 0, else the codec embedding
// row of tok[r] (ids checked on the host).
__global__ void k_token_rows(DevQ4 w, const uint32_t *tok, const int *slot, const float *text, float *out, int H) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
    if (j >= H) return;
    const int s = slot[r];
    out[(size_t)r * H + j] = s >= 0 ? text[(size_t)s * H + j] : q4_element(w, tok[r], j);
}

void launch_token_rows(hipStream_t st, const DevQ4 &w, const uint32_t *tok, const int *slot, const float *text,
                       int rows, float *out, int H) {
    hipLaunchKernelGGL(k_token_rows, dim3((unsigned)((H + 255) / 256), (unsigned)rows), dim3(256), 0, st, w, tok, slot,
                       text, out, H);
}

// sample_argmax (src/code_predictor.rs:328-334) of each row: the last index
// of the maximum; a NaN sets *status (per row) to QTTS_ENAN and gives 0.
// With a table, the row also copies table[code] (width floats; zeros past
// table_rows) to rows_out + r * rows_ld.
__global__ __launch_bounds__(256) void k_argmax_rows(const float *logits, int n, uint32_t *out, long long out_stride,
                                                     int *status, long long status_stride, const float *table,
                                                     int table_rows, int width, float *rows_out, long long rows_ld) {
    __shared__ float sv[256];
    __shared__ int si[256];
    __shared__ int snan;
    const int r = blockIdx.x, tid = threadIdx.x;
    const float *row = logits + (size_t)r * n;
    if (tid == 0) snan = 0;
    __syncthreads();
    float bv = -INFINITY;
    int bi = -1, nan = 0;
    for (int i = tid; i < n; i += 256) {
        const float v = row[i];
        if (v != v)
            nan = 1;
        else if (bi < 0 || v >= bv) {
            bv = v;
            bi = i;
        }
    }
    if (nan) atomicOr(&snan, 1);
    sv[tid] = bv;
    si[tid] = bi;
    __syncthreads();
    for (int stp = 128; stp > 0; stp >>= 1) {
        if (tid < stp) {
            const float ov = sv[tid + stp];
            const int oi = si[tid + stp];
            if (oi >= 0 && (si[tid] < 0 || ov > sv[tid] || (ov == sv[tid] && oi > si[tid]))) {
                sv[tid] = ov;
                si[tid] = oi;
            }
        }
        __syncthreads();
    }
    const uint32_t code = snan ? 0u : (uint32_t)(si[0] < 0 ? 0 : si[0]);
    if (tid == 0) {
        out[(size_t)r * out_stride] = code;
        if (snan && status) *byte_off(status, (long long)r * status_stride) = QTTS_ENAN;
    }
    if (table) {
        const float *src = table + (size_t)code * width;
        for (int j = tid; j < width; j += 256)
            rows_out[(size_t)r * rows_ld + j] = code < (uint32_t)table_rows ? src[j] : 0.0f;
    }
}

void launch_argmax_rows(hipStream_t st, const float *logits, int rows, int n, uint32_t *out, long long out_stride,
                        int *status, long long status_stride, const float *table, int table_rows, int width,
                        float *rows_out, long long rows_ld) {
    hipLaunchKernelGGL(k_argmax_rows, dim3((unsigned)rows), dim3(256), 0, st, logits, n, out, out_stride, status,
                       status_stride, table, table_rows, width, rows_out, rows_ld);
}

// ---------------------------------------------------------------------------
// Upload-time repack: reference [K][N/2] + [K][N/32] -> panels [p0 + pl][K].
// ---------------------------------------------------------------------------
__global__ void k_repack(const uint8_t *packed, const uint16_t *scales, int K, int N, int p0, uint4 *wq,
                         uint16_t *ws) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t panels = (size_t)(N / 32);
    if (idx >= panels * (size_t)K) return;
    const size_t pl = idx / (size_t)K, k = idx - pl * (size_t)K;
    wq[((size_t)p0 + pl) * K + k] = *reinterpret_cast<const uint4 *>(packed + k * (size_t)(N / 2) + pl * 16);
    ws[((size_t)p0 + pl) * K + k] = scales[k * panels + pl];
}

void launch_repack_q4(hipStream_t st, const uint8_t *packed, const uint16_t *scales, int K, int N, int col0,
                      int Ntot, uint4 *wq, uint16_t *ws) {
    (void)Ntot;
    const size_t total = (size_t)(N / 32) * K;
    hipLaunchKernelGGL(k_repack, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, packed, scales, K, N,
                       col0 / 32, wq, ws);
}

}  // namespace qtts
