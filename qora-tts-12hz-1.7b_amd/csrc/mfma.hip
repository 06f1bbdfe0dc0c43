// mfma.hip — the Q4 GEMM on the matrix cores (v_mfma_f32_32x32x16_f16) for
// row counts where the VALU GEMV's per-row cost dominates: gemm_q4
// (src/gemv.rs:311-375) at M >= 8, and the talker prefill's projections
// (src/talker.rs:364-462).
//
// Exactness.  The reference forms every term as f32(f32(s)*x)*(nib-8) and
// sums in f32.  Here each term is (xh + xl) * (sa*q + sb*q) with
//   q = nib - 8 in [-8, 7], exact in binary16;
//   s = sa + sb, sa keeping the top 7 significand bits of the binary16 scale
//     and sb the low 4, so sa*q and sb*q are exact binary16 products
//     (formed with v_pk_mul_f16);
//   x = xh + xl, xh = f16(x), xl = f16(x - xh): |x - xh - xl| <= 2^-22 |x|.
// Products of binary16 values are exact in the f32 accumulator, and the
// xl*sb*q term (relative size 2^-18) is dropped, so every term carries a
// relative error of ~2^-18 or less before the f32 sums -- the f32 level the
// parity tolerance is set for.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.h"
#include "internal.h"

namespace qtts {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4v __attribute__((ext_vector_type(4)));

// Repack of one panel-major Q4 weight into the MFMA B-operand order
// (DevQ4Mfma in internal.h): thread (p, s, l) gathers its 8 nibbles.
// A scale of magnitude above 8188 would overflow binary16 in sa * q; such a
// weight sets *too_large and stays on the VALU path.
__global__ void k_repack_mfma(DevQ4 w, uint32_t *wm, uint16_t *sa, uint16_t *sb, int *too_large) {
    const int Ks = w.K / 16, panels = w.N / 32;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)panels * Ks * 64;
    if (idx < total) {
        const int l = (int)(idx & 63);
        const size_t ps = idx >> 6;
        const int p = (int)(ps / Ks), s = (int)(ps - (size_t)p * Ks);
        const int col = l & 31, k0 = 16 * s + 8 * (l >> 5);
        const uint8_t *rows = reinterpret_cast<const uint8_t *>(w.wq + (size_t)p * w.K);
        uint32_t word = 0;
        for (int i = 0; i < 8; i++) {
            const uint8_t b = rows[(size_t)(k0 + i) * 16 + (col >> 1)];
            const uint32_t nib = (col & 1) ? (b >> 4) : (b & 15u);
            word |= nib << (4 * (i >> 1) + 16 * (i & 1));
        }
        wm[idx] = word;
    }
    // scales: one thread per (panel, row)
    const size_t nrows = (size_t)panels * w.K;
    if (idx < nrows) {
        const uint16_t s = w.ws[idx];
        if (fabsf((float)__builtin_bit_cast(_Float16, s)) > 8188.0f) atomicOr(too_large, 1);
        const uint16_t hi = s & 0xFFF0u;  // top 7 significand bits (sign and exponent kept)
        sa[idx] = hi;
        const float d = (float)__builtin_bit_cast(_Float16, s) - (float)__builtin_bit_cast(_Float16, hi);
        sb[idx] = __builtin_bit_cast(uint16_t, (_Float16)d);  // exact
    }
}

// One block per row m < Mpad: v = the row after the prologue (plain,
// rms_norm_f16 of src/gemv.rs:406-417, or silu(g)*u of
// src/talker.rs:342-345, with the same expression order as the GEMV path),
// then v * 2^e split into binary16 hi + lo, with e the per-row exponent that
// puts max|v| * 2^e in [2^14, 2^15) (no binary16 overflow; small entries keep
// their relative precision).  With RMSNorm, max|v| is taken as
// (1/rms) * max|x * gamma| from the same reduction as the sum of squares (one
// block barrier, and the gammas load with the row), which can miss max|v| by
// a few ulps: e is then one lower, putting max|v| * 2^e in [2^13, 2^15).
// rexp[m] = e; rows >= M are zero with e = 0.  xh and xl are stored in the
// MFMA A-operand order -- [M-tile][16-row step][lane][8] -- so that each
// wave's operand load of a step is one contiguous KiB.
template <int G>  // 8-value groups per thread: K <= 2048 * G
__global__ __launch_bounds__(256) void k_mfma_rows(MfmaRowsParams P) {
    __shared__ float red[2][4];
    const int m = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = P.K, Ks = K / 16, ng = K / 8;
    // 8-value group g = k / 8 of row m goes to the A-operand slot of lane
    // (m % 32) + 32 (g % 2) in step g / 2 of M-tile m / 32
    const size_t tile = (size_t)(m >> 5) * Ks * 64 + (m & 31);
    if (m >= P.M) {
        for (int g = tid; g < ng; g += 256) {
            const size_t o = (tile + (size_t)(g >> 1) * 64 + 32 * (g & 1)) * 8;
            *reinterpret_cast<half8 *>(P.xh + o) = (half8){};
            *reinterpret_cast<half8 *>(P.xl + o) = (half8){};
        }
        if (tid == 0) P.rexp[m] = 0;
        return;
    }
    const float *src = P.x + (size_t)m * P.ldx;
    const bool norm = P.mode == MFMA_ROWS_RMSNORM;
    float v[G][8];
    uint32_t gw[G][4];
    // 1. the row's values and gammas (all loads first); the sum of squares
    //    and max|x * gamma| (RMSNorm) or max|v|
#pragma unroll
    for (int j = 0; j < G; j++) {
        const int g = tid + 256 * j;
        if (g < ng) {
            const float4 a = *reinterpret_cast<const float4 *>(src + 8 * g);
            const float4 b = *reinterpret_cast<const float4 *>(src + 8 * g + 4);
            v[j][0] = a.x, v[j][1] = a.y, v[j][2] = a.z, v[j][3] = a.w;
            v[j][4] = b.x, v[j][5] = b.y, v[j][6] = b.z, v[j][7] = b.w;
            if (norm) {
                const uint4 q = *reinterpret_cast<const uint4 *>(P.gamma + 8 * g);
                gw[j][0] = q.x, gw[j][1] = q.y, gw[j][2] = q.z, gw[j][3] = q.w;
            }
            if (P.mode == MFMA_ROWS_SWIGLU) {
                const float4 c = *reinterpret_cast<const float4 *>(src + K + 8 * g);
                const float4 d = *reinterpret_cast<const float4 *>(src + K + 8 * g + 4);
                const float u[8] = {c.x, c.y, c.z, c.w, d.x, d.y, d.z, d.w};
#pragma unroll
                for (int i = 0; i < 8; i++) v[j][i] = (v[j][i] / (1.0f + expf(-v[j][i]))) * u[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[j][i] = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; q++) gw[j][q] = 0u;
        }
    }
    float ss = 0.0f, mx = 0.0f;
#pragma unroll
    for (int j = 0; j < G; j++)
#pragma unroll
        for (int i = 0; i < 8; i++) {
            ss += v[j][i] * v[j][i];
            // NaN entries drop out of the max here and stay NaN below
            mx = fmaxf(mx, fabsf(norm ? v[j][i] * f16_to_f32((uint16_t)(gw[j][i / 2] >> (16 * (i & 1)))) : v[j][i]));
        }
    ss = wave_sum(ss);
    mx = wave_max(mx);
    if (lane == 0) {
        red[0][wave] = ss;
        red[1][wave] = mx;
    }
    __syncthreads();
    mx = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
    if (norm) {
        ss = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
        const float inv = 1.0f / sqrtf(ss / (float)K + 1e-6f);
        mx *= inv;
#pragma unroll
        for (int j = 0; j < G; j++)
#pragma unroll
            for (int i = 0; i < 8; i++) v[j][i] = v[j][i] * inv * f16_to_f32((uint16_t)(gw[j][i / 2] >> (16 * (i & 1))));
    }
    // 2. the row exponent
    int e = 0;
    if (mx > 0.0f && mx < INFINITY) {
        int E;
        (void)frexpf(mx, &E);  // mx = f * 2^E, f in [0.5, 1)
        e = min((norm ? 14 : 15) - E, 126);
    }
    if (tid == 0) P.rexp[m] = e;
    if (P.norm_out) {
#pragma unroll
        for (int j = 0; j < G; j++) {
            const int g = tid + 256 * j;
            if (g >= ng) continue;
            float *dst = P.norm_out + (size_t)m * P.ldn + 8 * g;
#pragma unroll
            for (int i = 0; i < 8; i++) dst[i] = v[j][i];
        }
    }
    // 3. the binary16 hi + lo split
#pragma unroll
    for (int j = 0; j < G; j++) {
        const int g = tid + 256 * j;
        if (g >= ng) continue;
        half8 h, l;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float s = ldexpf(v[j][i], e);
            h[i] = (_Float16)s;
            l[i] = (_Float16)(s - (float)h[i]);
        }
        const size_t o = (tile + (size_t)(g >> 1) * 64 + 32 * (g & 1)) * 8;
        *reinterpret_cast<half8 *>(P.xh + o) = h;
        *reinterpret_cast<half8 *>(P.xl + o) = l;
    }
}

// One 32-column panel x one K chunk of 4 * SW 16-row steps per block; wave w
// takes steps [w * SW, (w + 1) * SW) of the chunk and issues all of their
// operand loads before its first MFMA (a step past K re-reads the last step
// and contributes zero: its scales are masked).  MT M-tiles of 32 rows share
// each step's B operand.  The waves are summed through LDS; with several
// chunks, each block stores its tile to `part` and the last block of a panel
// to arrive (a counter per panel) adds the chunks in chunk order --
// deterministic -- and finishes: * 2^-rexp[m], + bias, store or accumulate.
template <int MT, int SW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_gemm_mfma(GemmMfmaParams P) {
    __shared__ float red[4][MT * 1024];
    __shared__ int s_last;
    const int p = blockIdx.x, ch = blockIdx.y, kc = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = P.w.K, N = P.w.N, Ks = K / 16, Mpad = 32 * MT;
    const int s0 = (ch * 4 + wave) * SW;
    const int half = lane >> 5, col = lane & 31;

    // 1. every operand of this wave's steps
    uint32_t wq[SW];
    u32x4v sav[SW], sbv[SW];
    half8 xh[SW][MT], xl[SW][MT];
#pragma unroll
    for (int i = 0; i < SW; i++) {
        const int s = min(s0 + i, Ks - 1);
        const int krow = 16 * s + 8 * half;
        wq[i] = P.w.wm[((size_t)p * Ks + s) * 64 + lane];
        sav[i] = *reinterpret_cast<const u32x4v *>(P.w.sa + (size_t)p * K + krow);
        sbv[i] = *reinterpret_cast<const u32x4v *>(P.w.sb + (size_t)p * K + krow);
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const size_t off = (((size_t)t * Ks + s) * 64 + lane) * 8;
            xh[i][t] = *reinterpret_cast<const half8 *>(P.xh + off);
            xl[i][t] = *reinterpret_cast<const half8 *>(P.xl + off);
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first wait
    f32x16 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
    // 2. B = (sa + sb) * q as two exact binary16 operands; three MFMAs per tile
#pragma unroll
    for (int i = 0; i < SW; i++) {
        const bool in = s0 + i < Ks;
        half8 ba, bb;
        const uint32_t sap[4] = {sav[i].x, sav[i].y, sav[i].z, sav[i].w};
        const uint32_t sbp[4] = {sbv[i].x, sbv[i].y, sbv[i].z, sbv[i].w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // rows 2j, 2j+1 as binary16 1024 + nib (magic exponent), minus 1032
            typedef _Float16 half2v __attribute__((ext_vector_type(2)));
            const uint32_t bits = ((wq[i] >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
            const half2v q = __builtin_bit_cast(half2v, bits) - (half2v){(_Float16)1032.0f, (_Float16)1032.0f};
            const half2v a = q * __builtin_bit_cast(half2v, in ? sap[j] : 0u);
            const half2v b = q * __builtin_bit_cast(half2v, in ? sbp[j] : 0u);
            ba[2 * j] = a.x;
            ba[2 * j + 1] = a.y;
            bb[2 * j] = b.x;
            bb[2 * j + 1] = b.y;
        }
#pragma unroll
        for (int t = 0; t < MT; t++) {
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh[i][t], ba, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh[i][t], bb, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl[i][t], ba, acc[t], 0, 0, 0);
        }
    }
    // 3. the 4 waves through LDS.  D layout: lane l, register r -> row
    //    (r/4)*8 + (l/32)*4 + r%4, column l%32
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) red[wave][t * 1024 + ((r >> 2) * 8 + half * 4 + (r & 3)) * 32 + col] = acc[t][r];
    __syncthreads();
    const int M = P.M;
    if (kc > 1) {
        float *mine = P.part + (size_t)ch * Mpad * N;
        for (int i = tid; i < M * 32; i += 256) {
            const int m = i >> 5, n = 32 * p + (i & 31);
            st_dev(&mine[(size_t)m * N + n], (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]));
        }
        wait_stores();
        __syncthreads();
        if (tid == 0) s_last = arrive_dev(&P.counters[p]) == (unsigned)(kc - 1);
        __syncthreads();
        if (!s_last) return;
        if (tid == 0) reset_dev(&P.counters[p]);
    }
    // the block's outputs i = tid + 256 u; with several chunks, the partials
    // of 4 chunks for all of a thread's outputs are loaded before any is
    // added (in chunk order)
    constexpr int U = MT * 4;
    float v[U];
    if (kc > 1) {
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = 0.0f;
        uint32_t off[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = tid + 256 * u;
            off[u] = (uint32_t)min(i >> 5, M - 1) * (uint32_t)N + (uint32_t)(32 * p + (i & 31));
        }
        for (int c0 = 0; c0 < kc; c0 += 4) {
            float t[4][U];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float *pc = P.part + (size_t)min(c0 + j, kc - 1) * Mpad * N;  // uniform
#pragma unroll
                for (int u = 0; u < U; u++) t[j][u] = ld_dev(pc + off[u]);
            }
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int u = 0; u < U; u++)
                    if (c0 + j < kc) v[u] += t[j][u];
        }
    } else {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = tid + 256 * u;
            v[u] = (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
        }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int i = tid + 256 * u, m = i >> 5, n = 32 * p + (i & 31);
        if (m >= M) continue;
        float r = ldexpf(v[u], -P.rexp[m]);
        if (P.bias) r += P.bias[n];
        float *dst = P.y + (size_t)m * P.ldy + n;
        *dst = P.accumulate ? *dst + r : r;
    }
}

}  // namespace

void launch_repack_mfma(hipStream_t st, const DevQ4 &w, uint32_t *wm, uint16_t *sa, uint16_t *sb, int *too_large) {
    const size_t total = (size_t)(w.N / 32) * (w.K / 16) * 64;
    const size_t nrows = (size_t)(w.N / 32) * w.K;
    const size_t n = total > nrows ? total : nrows;
    hipLaunchKernelGGL(k_repack_mfma, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, wm, sa, sb, too_large);
}

void launch_mfma_rows(hipStream_t st, const MfmaRowsParams &p) {
    const int g = (p.K / 8 + 255) / 256;
    if (g <= 1)
        hipLaunchKernelGGL(k_mfma_rows<1>, dim3((unsigned)p.Mpad), dim3(256), 0, st, p);
    else if (g == 2)
        hipLaunchKernelGGL(k_mfma_rows<2>, dim3((unsigned)p.Mpad), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(k_mfma_rows<4>, dim3((unsigned)p.Mpad), dim3(256), 0, st, p);
}

template <int MT>
static void launch_gemm_mfma_mt(hipStream_t st, const GemmMfmaParams &p, int sw, int kc) {
    const dim3 grid((unsigned)(p.w.N / 32), (unsigned)kc);
    switch (sw) {
        case 8: hipLaunchKernelGGL((k_gemm_mfma<MT, 8>), grid, dim3(256), 0, st, p); break;
        case 4: hipLaunchKernelGGL((k_gemm_mfma<MT, 4>), grid, dim3(256), 0, st, p); break;
        case 2: hipLaunchKernelGGL((k_gemm_mfma<MT, 2>), grid, dim3(256), 0, st, p); break;
        default: hipLaunchKernelGGL((k_gemm_mfma<MT, 1>), grid, dim3(256), 0, st, p); break;
    }
}

void launch_gemm_mfma(hipStream_t st, const GemmMfmaParams &p, int mt, int sw, int kc) {
    if (mt == 1)
        launch_gemm_mfma_mt<1>(st, p, sw, kc);
    else
        launch_gemm_mfma_mt<2>(st, p, sw, kc);
}

}  // namespace qtts
