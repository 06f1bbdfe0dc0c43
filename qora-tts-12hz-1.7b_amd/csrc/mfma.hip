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
__global__ void k_repack_mfma(DevQ4 w, uint32_t *wm, uint16_t *sa, uint16_t *sb) {
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
        const uint16_t hi = s & 0xFFF0u;  // top 7 significand bits (sign and exponent kept)
        sa[idx] = hi;
        const float d = (float)__builtin_bit_cast(_Float16, s) - (float)__builtin_bit_cast(_Float16, hi);
        sb[idx] = __builtin_bit_cast(uint16_t, (_Float16)d);  // exact
    }
}

// xh[m][k] = f16(x), xl[m][k] = f16(x - xh) for m < M; rows M .. Mpad-1 zero.
__global__ void k_split_x(const float *x, int M, int ldx, int K, int Mpad, _Float16 *xh, _Float16 *xl) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)Mpad * K) return;
    const int m = (int)(idx / K), k = (int)(idx - (size_t)m * K);
    float v = m < M ? x[(size_t)m * ldx + k] : 0.0f;
    const _Float16 h = (_Float16)v;
    xh[idx] = h;
    xl[idx] = (_Float16)(v - (float)h);
}

// One 32-column panel x one K chunk per block; the 4 waves take consecutive
// quarters of the chunk's 16-row steps and are summed through LDS.  MT
// M-tiles of 32 rows share each step's B operand.
template <int MT>
__global__ __launch_bounds__(256) void k_gemm_mfma(GemmMfmaParams P) {
    __shared__ float red[4][MT * 1024];
    const int p = blockIdx.x, ch = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = P.w.K, Ks = K / 16, Mpad = 32 * MT;
    const int per_wave = P.steps / 4;
    const int s0 = ch * P.steps + wave * per_wave, s1 = min(Ks, s0 + per_wave);
    f32x16 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
    const int half = lane >> 5, col = lane & 31;
    for (int s = s0; s < s1; s++) {
        const int krow = 16 * s + 8 * half;
        const uint32_t w = P.w.wm[((size_t)p * Ks + s) * 64 + lane];
        const u32x4v sa = *reinterpret_cast<const u32x4v *>(P.w.sa + (size_t)p * K + krow);
        const u32x4v sb = *reinterpret_cast<const u32x4v *>(P.w.sb + (size_t)p * K + krow);
        half8 xh[MT], xl[MT];
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const size_t off = (size_t)(32 * t + col) * K + krow;
            xh[t] = *reinterpret_cast<const half8 *>(P.xh + off);
            xl[t] = *reinterpret_cast<const half8 *>(P.xl + off);
        }
        // q pairs (rows 2j, 2j+1) as binary16: 1024 + nib from the magic
        // exponent, minus 1032
        half8 ba, bb;
        const uint32_t sap[4] = {sa.x, sa.y, sa.z, sa.w}, sbp[4] = {sb.x, sb.y, sb.z, sb.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t bits = ((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
            typedef _Float16 half2v __attribute__((ext_vector_type(2)));
            const half2v q = __builtin_bit_cast(half2v, bits) - (half2v){(_Float16)1032.0f, (_Float16)1032.0f};
            const half2v a = q * __builtin_bit_cast(half2v, sap[j]);
            const half2v b = q * __builtin_bit_cast(half2v, sbp[j]);
            ba[2 * j] = a.x;
            ba[2 * j + 1] = a.y;
            bb[2 * j] = b.x;
            bb[2 * j + 1] = b.y;
        }
#pragma unroll
        for (int t = 0; t < MT; t++) {
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh[t], ba, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh[t], bb, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl[t], ba, acc[t], 0, 0, 0);
        }
    }
    // D layout: lane l, register r -> row (r/4)*8 + (l/32)*4 + r%4, column l%32
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) red[wave][t * 1024 + ((r >> 2) * 8 + half * 4 + (r & 3)) * 32 + col] = acc[t][r];
    __syncthreads();
    float *out = P.part + (size_t)ch * Mpad * P.w.N;
    for (int i = tid; i < MT * 1024; i += 256) {
        const int m = i >> 5, n = i & 31;
        out[(size_t)m * P.w.N + 32 * p + n] = (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
    }
}

// y[m][n] (+)= sum over chunks (+ bias[n]), m < M.
__global__ void k_gemm_reduce(const float *part, int kc, int M, int Mpad, int N, const float *bias, float *y, int ldy,
                              int accumulate) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)M * N) return;
    const int m = (int)(idx / N), n = (int)(idx - (size_t)m * N);
    float v = 0.0f;
    for (int c = 0; c < kc; c++) v += part[((size_t)c * Mpad + m) * N + n];
    if (bias) v += bias[n];
    float *dst = y + (size_t)m * ldy + n;
    *dst = accumulate ? *dst + v : v;
}

}  // namespace

void launch_repack_mfma(hipStream_t st, const DevQ4 &w, uint32_t *wm, uint16_t *sa, uint16_t *sb) {
    const size_t total = (size_t)(w.N / 32) * (w.K / 16) * 64;
    const size_t nrows = (size_t)(w.N / 32) * w.K;
    const size_t n = total > nrows ? total : nrows;
    hipLaunchKernelGGL(k_repack_mfma, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, wm, sa, sb);
}

void launch_split_x(hipStream_t st, const float *x, int M, int ldx, int K, int Mpad, _Float16 *xh, _Float16 *xl) {
    const size_t n = (size_t)Mpad * K;
    hipLaunchKernelGGL(k_split_x, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, M, ldx, K, Mpad, xh, xl);
}

void launch_gemm_mfma(hipStream_t st, const GemmMfmaParams &p, int mt, int kc) {
    const dim3 grid((unsigned)(p.w.N / 32), (unsigned)kc);
    if (mt == 1)
        hipLaunchKernelGGL(k_gemm_mfma<1>, grid, dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(k_gemm_mfma<2>, grid, dim3(256), 0, st, p);
}

void launch_gemm_reduce(hipStream_t st, const float *part, int kc, int M, int Mpad, int N, const float *bias, float *y,
                        int ldy, int accumulate) {
    const size_t n = (size_t)M * N;
    hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, kc, M, Mpad, N, bias,
                       y, ldy, accumulate);
}

}  // namespace qtts
