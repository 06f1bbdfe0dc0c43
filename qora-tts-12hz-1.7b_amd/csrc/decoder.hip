// decoder.hip — the speech decoder's kernels (decode_to_audio,
// src/decoder.rs:394-509), all f32 like the reference.
//
//  k_dec_gather   codebook rows of every frame: group 0's, and the sum of
//                 the other groups' in group order (src/decoder.rs:142-189)
//  k_dec_rmsnorm  rms_norm_f32 per frame (src/decoder.rs:515-525)
//  k_dec_rope     apply_rope_split_half of q and k (src/decoder.rs:556-578)
//  k_dec_attn     causal sliding-window attention, one wave per (frame, head)
//  k_dec_swiglu   silu(gate) * up
//  k_dec_dwconv   causal depthwise convolution (src/conv.rs:280-345)
//  k_dec_lnorm    channel-first LayerNorm per time step, channels summed in
//                 order (src/decoder.rs:580-602); k_dec_lnorm_tile the same
//                 over an LDS tile of 16 or 8 time steps
//  k_dec_snake    SnakeBeta (src/conv.rs:347-400), optionally recording
//                 max |out| for the convolution that reads it
//  k_dec_conv_mfma  every projection and convolution on the matrix cores
//                 (v_mfma_f32_32x32x16_f16 with binary16 hi + lo operands):
//                 causal convolutions as implicit GEMMs, one output phase
//                 of a transposed convolution, linear layers as one tap;
//                 fused epilogues; k_dec_conv_win for convolutions of 3+
//                 taps (the input window split once into LDS; the variant
//                 k_dec_conv_win_tw, one channel tile per wave, at 3 and 4
//                 tiles),
//                 k_dec_conv_mfma_ks for launches too small to fill the GPU
//  k_dec_absmax   max |x| of a layer input (the operand scale)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <cstdint>

#include "device_common.h"
#include "internal.h"

namespace qtts {

namespace {

constexpr unsigned kSnakeBlocks = 8192;  // SnakeBeta grid size target (threads stride through their channel)
// Matrix-core launches of fewer blocks than this at one channel tile split
// K over a block's waves instead (measured: 1,024 ahead of 0 and 4,096).
constexpr size_t kDecFillBlocks = 1024;


__global__ void k_dec_gather(DecGatherParams P) {
    const int t = blockIdx.x, cd = P.cd;
    for (int d = threadIdx.x; d < cd; d += blockDim.x) {
        uint32_t c0 = P.codes[t];
        if (c0 >= (uint32_t)P.cb_size) {
            if (d == 0) atomicOr(P.status, 1);
            c0 = 0;
        }
        P.e0[(size_t)t * cd + d] = P.first[(size_t)c0 * cd + d];
        float s = 0.0f;
        for (int g = 0; g < P.num_rest; g++) {
            uint32_t c = P.codes[(size_t)(g + 1) * P.ld + t];
            if (c >= (uint32_t)P.cb_size) {
                if (d == 0) atomicOr(P.status, 1);
                c = 0;
            }
            s += P.rest[g][(size_t)c * cd + d];
        }
        P.es[(size_t)t * cd + d] = s;
    }
}

// GELU, the tanh form the reference uses.
__device__ __forceinline__ float dec_gelu(float x) { return x * 0.5f * (1.0f + tanhf(x * 0.7071067811865476f)); }

// rms_norm_f32 of each of `rows` rows of n values: one block per row.
__global__ __launch_bounds__(256) void k_dec_rmsnorm(const float *x, const float *gamma, int n, float eps, float *out) {
    __shared__ float red[4];
    const float *r = x + (size_t)blockIdx.x * n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) ss += r[i] * r[i];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) out[(size_t)blockIdx.x * n + i] = r[i] * inv * gamma[i];
}

// Split-half rotation of q and k at position = frame; no rotation past the
// table.  One thread per (frame, head, pair).
__global__ void k_dec_rope(float *q, float *k, int T, int heads, int hd, const float *cs, const float *sn, int rows,
                           int ld) {
    const int half = hd / 2;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)T * heads * half) return;
    const int i = (int)(idx % half), h = (int)(idx / half % heads), t = (int)(idx / half / heads);
    if (t >= rows) return;
    const float c = cs[(size_t)t * half + i], s = sn[(size_t)t * half + i];
    float *qb = q + (size_t)t * ld + (size_t)h * hd, *kb = k + (size_t)t * ld + (size_t)h * hd;
    float x0 = qb[i], x1 = qb[half + i];
    qb[i] = x0 * c - x1 * s;
    qb[half + i] = x1 * c + x0 * s;
    x0 = kb[i], x1 = kb[half + i];
    kb[i] = x0 * c - x1 * s;
    kb[half + i] = x1 * c + x0 * s;
}

// Causal sliding-window attention (src/decoder.rs:248-275): one wave per
// (frame t, head h); scores over positions max(0, t+1-window) .. t, softmax,
// then out[d] = sum over positions in order of p * v[d] (lane = d).
__global__ __launch_bounds__(256) void k_dec_attn(DecAttnParams P) {
    __shared__ float ps[4][kDecMaxWindow];
    __shared__ float qs[4][kDecMaxHeadDim];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int pair = blockIdx.x * 4 + wave;
    const bool valid = pair < P.T * P.heads;  // wave-uniform; every wave reaches both barriers
    const int t = valid ? pair / P.heads : 0, h = valid ? pair - t * P.heads : 0;
    const int ad = P.heads * P.hd, ld = P.ld > 0 ? P.ld : ad;
    const int start = t + 1 > P.window ? t + 1 - P.window : 0, n = t + 1 - start;
    if (valid)
        for (int d = lane; d < P.hd; d += 64) qs[wave][d] = P.q[(size_t)t * ld + (size_t)h * P.hd + d];
    __syncthreads();
    float inv = 0.0f;
    if (valid) {
        float mx = -INFINITY;
        for (int s = lane; s < n; s += 64) {
            const float *k = P.k + (size_t)(start + s) * ld + (size_t)h * P.hd;
            float dot = 0.0f;
            for (int d = 0; d < P.hd; d++) dot += qs[wave][d] * k[d];
            dot *= P.scale;
            ps[wave][s] = dot;
            mx = fmaxf(mx, dot);
        }
        mx = wave_max(mx);
        float sum = 0.0f;
        for (int s = lane; s < n; s += 64) {
            const float e = expf(ps[wave][s] - mx);
            ps[wave][s] = e;
            sum += e;
        }
        inv = 1.0f / wave_sum(sum);
    }
    __syncthreads();
    if (valid)
        for (int d = lane; d < P.hd; d += 64) {
            float o = 0.0f;
            for (int s = 0; s < n; s++) o += (ps[wave][s] * inv) * P.v[(size_t)(start + s) * ld + (size_t)h * P.hd + d];
            P.out[(size_t)t * ad + (size_t)h * P.hd + d] = o;
        }
}

__global__ void k_dec_swiglu(const float *g, const float *u, int rows, int width, int ld, float *out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * width) return;
    const size_t t = i / width, j = i - t * width, a = t * ld + j;
    out[i] = (g[a] / (1.0f + expf(-g[a]))) * u[a];
}

// Causal depthwise convolution (padding kernel_size - 1), channel-first.
__global__ void k_dec_dwconv(const float *x, const float *w, const float *b, int ch, int len, int ks, float *out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)ch * len) return;
    const int c = (int)(i / len), o = (int)(i - (size_t)c * len);
    float s = b[c];
    for (int k = 0; k < ks; k++) {
        const int p = o + k - (ks - 1);
        if (p >= 0) s += x[(size_t)c * len + p] * w[(size_t)c * ks + k];
    }
    out[i] = s;
}

// LayerNorm across channels at each time step (one thread per step; the
// channel sums run in channel order, 8 channels' loads issued together).
__global__ __launch_bounds__(64) void k_dec_lnorm(const float *x, const float *g, const float *b, int ch, int len,
                                                  float eps, float *out) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= len) return;
    const float *xt = x + t;
    float mean = 0.0f;
    int c = 0;
    for (; c + 8 <= ch; c += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = xt[(size_t)(c + i) * len];
#pragma unroll
        for (int i = 0; i < 8; i++) mean += v[i];
    }
    for (; c < ch; c++) mean += xt[(size_t)c * len];
    mean /= (float)ch;
    float var = 0.0f;
    for (c = 0; c + 8 <= ch; c += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = xt[(size_t)(c + i) * len];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float d = v[i] - mean;
            var += d * d;
        }
    }
    for (; c < ch; c++) {
        const float d = xt[(size_t)c * len] - mean;
        var += d * d;
    }
    const float inv = 1.0f / sqrtf(var / (float)ch + eps);
    for (c = 0; c < ch; c++) out[(size_t)c * len + t] = (xt[(size_t)c * len] - mean) * inv * g[c] + b[c];
}

// The same LayerNorm with TS time steps per block: the block's [ch][TS]
// input tile is loaded once into LDS (TS consecutive steps of a channel are
// consecutive addresses, 16 loads per thread in flight), thread t < TS runs
// step t's two channel sums in channel order from LDS -- the arithmetic of
// k_dec_lnorm, so the output is the same bit for bit -- and every thread
// writes the normalised tile.  One global round trip instead of one per 8
// channels of each pass.
template <int TS>
__global__ __launch_bounds__(256) void k_dec_lnorm_tile(const float *x, const float *g, const float *b, int ch, int len,
                                                        float eps, float *out) {
    extern __shared__ float tile[];  // [ch][TS]
    __shared__ float s_mean[TS], s_inv[TS];
    constexpr int U = 16;
    const int t0 = blockIdx.x * TS, tid = threadIdx.x;
    const int n = min(TS, len - t0);
    const int total = ch * TS;
    for (int base = 0; base < total; base += 256 * U) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * 256 + tid, c = i / TS, j = i - c * TS;
            v[u] = i < total && j < n ? x[(size_t)c * len + t0 + j] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int i = base + u * 256 + tid;
            if (i < total) tile[i] = v[u];
        }
    }
    __syncthreads();
    if (tid < n) {
        float mean = 0.0f;
        for (int c = 0; c < ch; c++) mean += tile[c * TS + tid];
        mean /= (float)ch;
        float var = 0.0f;
        for (int c = 0; c < ch; c++) {
            const float d = tile[c * TS + tid] - mean;
            var += d * d;
        }
        s_mean[tid] = mean;
        s_inv[tid] = 1.0f / sqrtf(var / (float)ch + eps);
    }
    __syncthreads();
    for (int i = tid; i < total; i += 256) {
        const int c = i / TS, j = i - c * TS;
        if (j < n) out[(size_t)c * len + t0 + j] = (tile[i] - s_mean[j]) * s_inv[j] * g[c] + b[c];
    }
}

// With add set, the input is x + add, stored to sum (which may be x: each
// element is read before it is written, by the same thread) before the
// activation: a residual sum made where it is next read.
// x + exp(-beta) * sin(exp(alpha) * x)^2 per channel, channel-first: block
// row y is channel y (its two exponentials computed once per thread, no
// division per element), and the blocks of a row stride through its
// samples.  With amax set, each block's largest |out| (NaN excluded) is
// folded into amax[block % kDecMaxSlots] by an unsigned atomicMax of the
// float bits, which orders non-negative floats as their values: the slots'
// maximum does not depend on the order of the blocks, and 64 slots keep the
// atomics from queueing on one address.
__global__ __launch_bounds__(256) void k_dec_snake(const float *x, const float *alpha, const float *beta, int ch,
                                                   int len, float *out, unsigned *amax, const float *add, float *sum) {
    const int c = blockIdx.y;
    const float a = expf(alpha[c]), inv_b = expf(-beta[c]);
    const size_t base = (size_t)c * len;
    float m = 0.0f;
    auto snake = [&](float v) {
        const float s = sinf(a * v);
        const float o = v + inv_b * s * s;
        m = fmaxf(m, fabsf(o));  // a NaN o leaves m as it was
        return o;
    };
    const int stride = gridDim.x * blockDim.x;
    if ((len & 3) == 0) {
        // rows of a multiple of 4 samples (every decoder stage): 16-byte
        // loads and stores, two in flight per thread
        const float4 *x4 = reinterpret_cast<const float4 *>(x + base);
        float4 *o4 = reinterpret_cast<float4 *>(out + base);
        const float4 *a4 = reinterpret_cast<const float4 *>(add + base);
        float4 *s4 = reinterpret_cast<float4 *>(sum + base);
        auto in = [&](int i) {  // x, or x + add stored to sum first
            float4 v = x4[i];
            if (add) {
                const float4 d = a4[i];
                v = make_float4(v.x + d.x, v.y + d.y, v.z + d.z, v.w + d.w);
                s4[i] = v;
            }
            return v;
        };
        const int n4 = len >> 2;
        int t = blockIdx.x * blockDim.x + threadIdx.x;
        for (; t + stride < n4; t += 2 * stride) {
            const float4 v0 = in(t), v1 = in(t + stride);
            o4[t] = make_float4(snake(v0.x), snake(v0.y), snake(v0.z), snake(v0.w));
            o4[t + stride] = make_float4(snake(v1.x), snake(v1.y), snake(v1.z), snake(v1.w));
        }
        if (t < n4) {
            const float4 v0 = in(t);
            o4[t] = make_float4(snake(v0.x), snake(v0.y), snake(v0.z), snake(v0.w));
        }
    } else {
        for (int t = blockIdx.x * blockDim.x + threadIdx.x; t < len; t += stride) {
            float v = x[base + t];
            if (add) {
                v += add[base + t];
                sum[base + t] = v;
            }
            out[base + t] = snake(v);
        }
    }
    if (!amax) return;  // uniform
    __shared__ float red[4];
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        atomicMax(&amax[(blockIdx.y * gridDim.x + blockIdx.x) % kDecMaxSlots], __float_as_uint(m));
    }
}

__global__ void k_dec_fill_u32(unsigned *p, int n, unsigned v) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// max |x| of n values into the kDecMaxSlots slots of amax, as k_dec_snake
// records it (for inputs of the matrix-core layers that no SnakeBeta makes).
__global__ __launch_bounds__(256) void k_dec_absmax(const float *x, size_t n, unsigned *amax) {
    float m = 0.0f;
    const size_t stride = (size_t)gridDim.x * blockDim.x, t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if ((n & 3) == 0 && ((uintptr_t)x & 15) == 0) {
        // 16-byte loads, four in flight per thread
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        const size_t n4 = n >> 2;
#pragma unroll 4
        for (size_t i = t0; i < n4; i += stride) {
            const float4 v = x4[i];
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    } else {
        for (size_t i = t0; i < n; i += stride) m = fmaxf(m, fabsf(x[i]));
    }
    __shared__ float red[4];
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        atomicMax(&amax[blockIdx.x % kDecMaxSlots], __float_as_uint(m));
    }
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// The exponent e that puts a positive finite maximum m at m * 2^e in
// [2^14, 2^15) (0 for zero, infinite or NaN).
__device__ __forceinline__ int split_exponent(float m) {
    if (!(m > 0.0f && m < INFINITY)) return 0;
    int E;
    (void)frexpf(m, &E);  // m = f * 2^E, f in [0.5, 1)
    return min(15 - E, 126);
}

// A convolution's weights as binary16 hi + lo MFMA A operands, scaled by
// 2^ew: thread (tile, step, lane) writes the 8 values of row
// m = 32 * tile + lane % 32 for step = (16-channel block cb, tap) with the
// taps inner (cb = step / taps, tap = step % taps), channels
// ci = 16 cb + 8 (lane / 32) + i (zero past M or cin): the element
// w[m * sm + ci * sci + k0 + tap * kd] -- for a causal convolution
// W[m][ci][tap] (src/conv.rs:114-184: sm = cin * ksize, sci = ksize, k0 = 0,
// kd = 1); for output phase r of a transposed one W[ci][m][r + (J-1-tap) s]
// (src/conv.rs:198-268: sm = ksize, sci = M * ksize, k0 = r + (J - 1) s,
// kd = -s), so that tap t reads the input J - 1 - t steps back.
// hi = f16(w'), lo = f16(w' - hi).
__global__ void k_dec_conv_repack(const float *w, long long sm, long long sci, int k0, int kd, int M, int cin,
                                  int taps, int cin16, int mtiles, int ksteps, int ew, _Float16 *wh, _Float16 *wl) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)mtiles * ksteps * 64) return;
    const int lane = (int)(idx & 63);
    const size_t ts = idx >> 6;
    const int tile = (int)(ts / ksteps), step = (int)(ts - (size_t)tile * ksteps);
    const int m = 32 * tile + (lane & 31), kb = 16 * step + 8 * (lane >> 5);
    const int cb = step / taps, tap = step - cb * taps;  // step = (16-channel block, tap), taps inner
    half8 h, l;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int ci = 16 * cb + (kb & 15) + i;
        const float v = (m < M && ci < cin && tap < taps)
                            ? ldexpf(w[(long long)m * sm + (long long)ci * sci + k0 + (long long)tap * kd], ew)
                            : 0.0f;
        const _Float16 hv = (_Float16)v;
        h[i] = hv;
        l[i] = (_Float16)(v - (float)hv);
    }
    reinterpret_cast<half8 *>(wh)[idx] = h;
    reinterpret_cast<half8 *>(wl)[idx] = l;
}

// A causal convolution c[m][n] = bias[m] + sum_{ci, tap} W[m][ci][tap] *
// x[ci][n + (tap - (ksize - 1)) * dilation] (zero before the signal) as an
// implicit GEMM on the matrix cores.  Each wave owns 32 output steps n and
// the block's MT tiles of 32 channels.  The A operands of a stage of
// kConvStage 16-row K steps are loaded once per block -- each wave loads a
// quarter of the (tile, step, hi/lo) units -- and staged in LDS (double
// buffered, one barrier per stage), so the four waves share them.  Per step
// each wave gathers its own B operand -- lane l: step n0 + l % 32, channels
// ci0 + 8 (l / 32) + i of one tap (a step is one tap of one block of 16
// channels, the taps of a block consecutive, so a tap re-reads the lines
// the previous step gathered, shifted by the dilation) -- scales
// it by 2^ex (ex from the producer's max |x|), splits it into binary16 hi +
// lo, and runs three MFMAs per tile: wh * xh + wh * xl + wl * xh.  Every
// product of binary16 values is exact in the f32 accumulator; the dropped
// wl * xl term and the two splits leave a relative error of about 2^-21 per
// term, the f32 level.  The next stage's operands are loaded before the
// current stage's MFMAs.
template <int MT, bool KF>  // KF: channels contiguous (sxc == 1, cin % 8 == 0)
__global__ __launch_bounds__(256) void k_dec_conv_mfma(DecConvMfmaParams P) {
    static_assert(kDecMaxSlots == 64, "one max slot per lane");
    constexpr int G = kConvStage;
    constexpr int UNITS = 2 * MT * G;  // 1-KiB operand units per stage: (step, tile, hi/lo)
    constexpr int UPW = UNITS / 4;     // per wave
    static_assert(UNITS % 4 == 0, "units split evenly over the 4 waves");
    __shared__ half8 As[2][UNITS][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int n = (blockIdx.x * 4 + wave) * 32 + col;  // this lane's output step
    const int t0 = blockIdx.y * MT;
    const int len = P.len, cin16 = P.cin16, ksteps = P.ksteps, nstage = ksteps / G;
    const bool multi = P.nphase > 1;  // uniform
    const _Float16 *wh = multi ? P.ph_wh[blockIdx.z] : P.wh, *wl = multi ? P.ph_wl[blockIdx.z] : P.wl;
    const int phase = multi ? (int)blockIdx.z : P.phase;
    // max |x| over the producer's slots, one per lane
    const int ex = split_exponent(wave_max(__uint_as_float(P.xmax[lane])));
    const float xs = ldexpf(1.0f, ex);
    const int cpl = P.cin - 8 * half;  // channels this lane's half may read at ci0 = 0

    // this wave's A units of stage g: unit u = (gs * MT + t) * 2 + hl
    auto load_a = [&](int g, half8 (&ua)[UPW]) {
#pragma unroll
        for (int k = 0; k < UPW; k++) {
            const int u = wave + 4 * k, hl = u & 1, t = (u >> 1) % MT, gs = (u >> 1) / MT;
            const size_t o = ((size_t)(t0 + t) * ksteps + g * G + gs) * 64 + lane;
            ua[k] = reinterpret_cast<const half8 *>(hl ? wl : wh)[o];
        }
    };
    // the 8 raw x values of this lane at step s (zero past the taps of a
    // padded last stage)
    auto load_b = [&](int s, float (&xv)[8]) {
        const int cb = s / P.ksize, tap = s - cb * P.ksize, ci0 = 16 * cb;  // wave-uniform
        const int p = n + (tap - (P.ksize - 1)) * P.dilation;
        const bool ok = n < len && p >= 0 && tap < P.ksize && ci0 < cpl;
        const float *xp = P.x + (long long)(ci0 + 8 * half) * P.sxc + (long long)(ok ? p : 0) * P.sxn;
        if constexpr (KF) {
            // all 8 channels exist (cin % 8 == 0): two 16-byte loads
            const float4 a = ok ? *reinterpret_cast<const float4 *>(xp) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 b = ok ? *reinterpret_cast<const float4 *>(xp + 4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            xv[0] = a.x, xv[1] = a.y, xv[2] = a.z, xv[3] = a.w;
            xv[4] = b.x, xv[5] = b.y, xv[6] = b.z, xv[7] = b.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) xv[i] = ok && ci0 + i < cpl ? xp[(long long)i * P.sxc] : 0.0f;
        }
    };
    f32x16 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
    half8 ua[UPW];
    float xv[G][8];
    load_a(0, ua);
#pragma unroll
    for (int gs = 0; gs < G; gs++) load_b(gs, xv[gs]);
#pragma unroll
    for (int k = 0; k < UPW; k++) As[0][wave + 4 * k][lane] = ua[k];
    __syncthreads();
    for (int g = 0; g < nstage; g++) {
        const int buf = g & 1;
        const bool more = g + 1 < nstage;  // uniform
        half8 na[UPW];
        float nx[G][8];
        if (more) {
            load_a(g + 1, na);
#pragma unroll
            for (int gs = 0; gs < G; gs++) load_b((g + 1) * G + gs, nx[gs]);
        }
#pragma unroll
        for (int gs = 0; gs < G; gs++) {
            half8 bh, bl;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float v = xv[gs][i] * xs;
                const _Float16 hv = (_Float16)v;
                bh[i] = hv;
                bl[i] = (_Float16)(v - (float)hv);
            }
#pragma unroll
            for (int t = 0; t < MT; t++) {
                const half8 ah = As[buf][(gs * MT + t) * 2][lane], al = As[buf][(gs * MT + t) * 2 + 1][lane];
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, acc[t], 0, 0, 0);
            }
        }
        if (more) {
            // buf ^ 1 was last read in stage g - 1, before the last barrier
#pragma unroll
            for (int k = 0; k < UPW; k++) As[buf ^ 1][wave + 4 * k][lane] = na[k];
#pragma unroll
            for (int gs = 0; gs < G; gs++)
#pragma unroll
                for (int i = 0; i < 8; i++) xv[gs][i] = nx[gs][i];
        }
        __syncthreads();
    }
    // D layout: lane l, register r -> row (r / 4) * 8 + (l / 32) * 4 + r % 4,
    // column l % 32
    if (n >= len) return;
    const int sc = -(ex + P.ew);
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = 32 * (t0 + t) + (r >> 2) * 8 + half * 4 + (r & 3);
            if (m >= P.M) continue;
            float v = ldexpf(acc[t][r], sc);
            if (P.bias) v += P.bias[m];
            if (P.act == DEC_ACT_GELU) v = dec_gelu(v);
            float *dst = P.c + (long long)m * P.ldc + (long long)n * P.out_stride + phase;
            switch (P.epi) {
                case DEC_EPI_STORE: *dst = v; break;
                case DEC_EPI_ACCUM: *dst += v; break;
                case DEC_EPI_SCALED_RESID: *dst += P.scale[m] * v; break;
                case DEC_EPI_RESID_IN: *dst = P.resid[dst - P.c] + (P.scale ? P.scale[m] * v : v); break;
                default: *dst = v < -1.0f ? -1.0f : (v > 1.0f ? 1.0f : v); break;  // DEC_EPI_CLAMP (NaN stays)
            }
        }
}

// The same product for launches too small to fill the GPU (the transformer's
// linears at 500 rows, the first Vocos stages): one block per (32 output
// steps, channel tile), its 4 waves splitting the K steps four ways (each
// wave loads its own A operands and gathers its own B), the partial sums
// added through LDS in wave order (deterministic) by wave 0, which runs the
// epilogue.  A quarter of the dependent step chain per wave and four times
// the blocks of k_dec_conv_mfma<1>.
template <bool KF>
__global__ __launch_bounds__(256) void k_dec_conv_mfma_ks(DecConvMfmaParams P) {
    static_assert(kDecMaxSlots == 64, "one max slot per lane");
    __shared__ float red[3][16][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int n = blockIdx.x * 32 + col;
    const int tile = blockIdx.y;
    const int len = P.len, ksteps = P.ksteps;
    const bool multi = P.nphase > 1;  // uniform
    const _Float16 *wh = multi ? P.ph_wh[blockIdx.z] : P.wh, *wl = multi ? P.ph_wl[blockIdx.z] : P.wl;
    const int phase = multi ? (int)blockIdx.z : P.phase;
    const int q = (ksteps + 3) / 4, s0 = wave * q, s1 = min(ksteps, s0 + q);
    const int ex = split_exponent(wave_max(__uint_as_float(P.xmax[lane])));
    const float xs = ldexpf(1.0f, ex);
    const int cpl = P.cin - 8 * half;
    auto load = [&](int s, half8 &ah, half8 &al, float (&xv)[8]) {
        const int cb = s / P.ksize, tap = s - cb * P.ksize, ci0 = 16 * cb;  // wave-uniform
        const int p = n + (tap - (P.ksize - 1)) * P.dilation;
        const bool ok = n < len && p >= 0 && ci0 < cpl;
        const float *xp = P.x + (long long)(ci0 + 8 * half) * P.sxc + (long long)(ok ? p : 0) * P.sxn;
        if constexpr (KF) {
            const float4 a = ok ? *reinterpret_cast<const float4 *>(xp) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const float4 b = ok ? *reinterpret_cast<const float4 *>(xp + 4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            xv[0] = a.x, xv[1] = a.y, xv[2] = a.z, xv[3] = a.w;
            xv[4] = b.x, xv[5] = b.y, xv[6] = b.z, xv[7] = b.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) xv[i] = ok && ci0 + i < cpl ? xp[(long long)i * P.sxc] : 0.0f;
        }
        const size_t o = ((size_t)tile * ksteps + s) * 64 + lane;
        ah = reinterpret_cast<const half8 *>(wh)[o];
        al = reinterpret_cast<const half8 *>(wl)[o];
    };
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    if (s0 < s1) {  // uniform
        half8 ah, al;
        float xv[8];
        load(s0, ah, al, xv);
        for (int s = s0; s < s1; s++) {
            half8 nh, nl;
            float nx[8];
            load(s + 1 < s1 ? s + 1 : s, nh, nl, nx);
            half8 bh, bl;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float v = xv[i] * xs;
                const _Float16 hv = (_Float16)v;
                bh[i] = hv;
                bl[i] = (_Float16)(v - (float)hv);
            }
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, acc, 0, 0, 0);
            ah = nh;
            al = nl;
#pragma unroll
            for (int i = 0; i < 8; i++) xv[i] = nx[i];
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < 16; r++) red[wave - 1][r][lane] = acc[r];
    }
    __syncthreads();
    if (wave > 0 || n >= len) return;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = ((acc[r] + red[0][r][lane]) + red[1][r][lane]) + red[2][r][lane];
    // D layout: lane l, register r -> row (r / 4) * 8 + (l / 32) * 4 + r % 4,
    // column l % 32
    const int sc = -(ex + P.ew);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = 32 * tile + (r >> 2) * 8 + half * 4 + (r & 3);
        if (m >= P.M) continue;
        float v = ldexpf(acc[r], sc);
        if (P.bias) v += P.bias[m];
        if (P.act == DEC_ACT_GELU) v = dec_gelu(v);
        float *dst = P.c + (long long)m * P.ldc + (long long)n * P.out_stride + phase;
        switch (P.epi) {
            case DEC_EPI_STORE: *dst = v; break;
            case DEC_EPI_ACCUM: *dst += v; break;
            case DEC_EPI_SCALED_RESID: *dst += P.scale[m] * v; break;
            case DEC_EPI_RESID_IN: *dst = P.resid[dst - P.c] + (P.scale ? P.scale[m] * v : v); break;
            default: *dst = v < -1.0f ? -1.0f : (v > 1.0f ? 1.0f : v); break;  // DEC_EPI_CLAMP (NaN stays)
        }
    }
}

// A causal convolution with 3 or more taps over a channel-first input
// (sxn == 1), its input window staged in LDS: per block of 16 input
// channels, the block's window -- positions n0 - (ksize - 1) * dilation ..
// n0 + 127 of those channels -- is loaded once (thread t: position t, the
// 16 channels' values, each load coalesced over the threads), scaled by 2^ex
// and split into binary16 hi + lo, and stored position-major per half of the
// channels ([8-channel half][position][8 channels], 16-byte rows, so the 16
// lanes of a 16-byte LDS read hit 16 consecutive rows: no bank conflicts),
// and every tap's B operand is two 16-byte LDS reads at position n - n0 +
// tap * dilation: each value is split once instead of once per tap.  The
// next channel block's window is loaded into registers during the current
// block's taps (double-buffered, one barrier per channel block); A operands
// come from global memory one step ahead.  Same operand order and products as k_dec_conv_mfma.
template <int MT>
__global__ __launch_bounds__(256) void k_dec_conv_win(DecConvMfmaParams P) {
    static_assert(kDecMaxSlots == 64, "one max slot per lane");
    constexpr int WMAX = 256;  // window positions: 128 + (ksize - 1) * dilation <= the block's threads
    __shared__ __align__(16) _Float16 wh_s[2][2][WMAX][8], wl_s[2][2][WMAX][8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int n0 = blockIdx.x * 128, n = n0 + wave * 32 + col;
    const int t0 = blockIdx.y * MT;
    const int len = P.len, ks = P.ksize, dil = P.dilation, ksteps = P.ksteps;
    const bool multi = P.nphase > 1;  // uniform
    const _Float16 *wh = multi ? P.ph_wh[blockIdx.z] : P.wh, *wl = multi ? P.ph_wl[blockIdx.z] : P.wl;
    const int phase = multi ? (int)blockIdx.z : P.phase;
    const int W = 128 + (ks - 1) * dil, wpos = n0 - (ks - 1) * dil + tid;  // this thread's window position
    const bool wok = tid < W && wpos >= 0 && wpos < len;
    const int ncb = P.cin16 / 16;
    const int ex = split_exponent(wave_max(__uint_as_float(P.xmax[lane])));
    const float xs = ldexpf(1.0f, ex);
    auto load_win = [&](int cb, float (&v)[16]) {
        const float *xp = P.x + (size_t)(16 * cb) * len + (wok ? wpos : 0);
#pragma unroll
        for (int c = 0; c < 16; c++) v[c] = wok && 16 * cb + c < P.cin ? xp[(size_t)c * len] : 0.0f;
    };
    auto store_win = [&](int buf, const float (&v)[16]) {
        if (tid >= W) return;
        half8 h[2], l[2];
#pragma unroll
        for (int c = 0; c < 16; c++) {
            const float x = v[c] * xs;
            const _Float16 hv = (_Float16)x;
            h[c >> 3][c & 7] = hv;
            l[c >> 3][c & 7] = (_Float16)(x - (float)hv);
        }
        *reinterpret_cast<half8 *>(&wh_s[buf][0][tid][0]) = h[0];
        *reinterpret_cast<half8 *>(&wh_s[buf][1][tid][0]) = h[1];
        *reinterpret_cast<half8 *>(&wl_s[buf][0][tid][0]) = l[0];
        *reinterpret_cast<half8 *>(&wl_s[buf][1][tid][0]) = l[1];
    };
    auto load_a = [&](int s, half8 (&ah)[MT], half8 (&al)[MT]) {
#pragma unroll
        for (int t = 0; t < MT; t++) {
            const size_t o = ((size_t)(t0 + t) * ksteps + s) * 64 + lane;
            ah[t] = reinterpret_cast<const half8 *>(wh)[o];
            al[t] = reinterpret_cast<const half8 *>(wl)[o];
        }
    };
    f32x16 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
    float wv[16];
    load_win(0, wv);
    store_win(0, wv);
    half8 ah[MT], al[MT];
    load_a(0, ah, al);
    __syncthreads();
    const int nsteps = ncb * ks;  // the steps past these (stage padding) hold zero weights
    for (int cb = 0; cb < ncb; cb++) {
        const int buf = cb & 1;
        const bool more = cb + 1 < ncb;  // uniform
        if (more) load_win(cb + 1, wv);
        for (int tap = 0; tap < ks; tap++) {
            const int s = cb * ks + tap;
            half8 nh[MT], nl[MT];
            load_a(s + 1 < nsteps ? s + 1 : s, nh, nl);
            const int p = wave * 32 + col + tap * dil;
            const half8 bh = *reinterpret_cast<const half8 *>(&wh_s[buf][half][p][0]);
            const half8 bl = *reinterpret_cast<const half8 *>(&wl_s[buf][half][p][0]);
#pragma unroll
            for (int t = 0; t < MT; t++) {
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[t], bh, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[t], bl, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[t], bh, acc[t], 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < MT; t++) {
                ah[t] = nh[t];
                al[t] = nl[t];
            }
        }
        // buf ^ 1 was last read in channel block cb - 1, before the last barrier
        if (more) store_win(buf ^ 1, wv);
        __syncthreads();
    }
    // D layout: lane l, register r -> row (r / 4) * 8 + (l / 32) * 4 + r % 4,
    // column l % 32
    if (n >= len) return;
    const int sc = -(ex + P.ew);
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = 32 * (t0 + t) + (r >> 2) * 8 + half * 4 + (r & 3);
            if (m >= P.M) continue;
            float v = ldexpf(acc[t][r], sc);
            if (P.bias) v += P.bias[m];
            if (P.act == DEC_ACT_GELU) v = dec_gelu(v);
            float *dst = P.c + (long long)m * P.ldc + (long long)n * P.out_stride + phase;
            switch (P.epi) {
                case DEC_EPI_STORE: *dst = v; break;
                case DEC_EPI_ACCUM: *dst += v; break;
                case DEC_EPI_SCALED_RESID: *dst += P.scale[m] * v; break;
                case DEC_EPI_RESID_IN: *dst = P.resid[dst - P.c] + (P.scale ? P.scale[m] * v : v); break;
                default: *dst = v < -1.0f ? -1.0f : (v > 1.0f ? 1.0f : v); break;  // DEC_EPI_CLAMP (NaN stays)
            }
        }
}

// k_dec_conv_win with the waves' roles swapped, for NW (3 or 4) channel
// tiles per block of NW waves: wave w owns channel tile NW * blockIdx.y + w
// -- its A operands loaded by it alone, where every wave of
// k_dec_conv_win<MT> loads all MT tiles' -- and all four 32-position tiles
// of the block, whose B operands it reads from the staged window (LDS,
// twice L1's bandwidth).  Per step a block reads NW * 2 KiB of A operands
// through L1 instead of 4 * NW * 2 KiB.  The window (up to 256 positions)
// is staged by the block's 64 * NW threads, position t + 64 * NW * q by
// thread t in pass q.  Same window, operands and product order per output
// as k_dec_conv_win: the same bits.
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_dec_conv_win_tw(DecConvMfmaParams P) {
    static_assert(kDecMaxSlots == 64, "one max slot per lane");
    constexpr int WMAX = 256, PT = 4;  // window positions; 32-position tiles per block
    constexpr int NT = 64 * NW, NP = (WMAX + NT - 1) / NT;  // threads; staging passes
    __shared__ __align__(16) _Float16 wh_s[2][2][WMAX][8], wl_s[2][2][WMAX][8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int n0 = blockIdx.x * 128;
    const int tile = blockIdx.y * NW + wave;  // < mtiles (the grid has mtiles / NW rows)
    const int len = P.len, ks = P.ksize, dil = P.dilation, ksteps = P.ksteps;
    const bool multi = P.nphase > 1;  // uniform
    const _Float16 *wh = multi ? P.ph_wh[blockIdx.z] : P.wh, *wl = multi ? P.ph_wl[blockIdx.z] : P.wl;
    const int phase = multi ? (int)blockIdx.z : P.phase;
    const int W = 128 + (ks - 1) * dil;  // window positions n0 - (ks - 1) * dil .. n0 + 127
    const int ncb = P.cin16 / 16;
    const int ex = split_exponent(wave_max(__uint_as_float(P.xmax[lane])));
    const float xs = ldexpf(1.0f, ex);
    auto load_win = [&](int cb, float (&v)[NP][16]) {
#pragma unroll
        for (int q = 0; q < NP; q++) {
            const int wi = tid + q * NT, wpos = n0 - (ks - 1) * dil + wi;
            const bool wok = wi < W && wpos >= 0 && wpos < len;
            const float *xp = P.x + (size_t)(16 * cb) * len + (wok ? wpos : 0);
#pragma unroll
            for (int c = 0; c < 16; c++) v[q][c] = wok && 16 * cb + c < P.cin ? xp[(size_t)c * len] : 0.0f;
        }
    };
    auto store_win = [&](int buf, const float (&v)[NP][16]) {
#pragma unroll
        for (int q = 0; q < NP; q++) {
            const int wi = tid + q * NT;
            if (wi >= W) continue;
            half8 h[2], l[2];
#pragma unroll
            for (int c = 0; c < 16; c++) {
                const float x = v[q][c] * xs;
                const _Float16 hv = (_Float16)x;
                h[c >> 3][c & 7] = hv;
                l[c >> 3][c & 7] = (_Float16)(x - (float)hv);
            }
            *reinterpret_cast<half8 *>(&wh_s[buf][0][wi][0]) = h[0];
            *reinterpret_cast<half8 *>(&wh_s[buf][1][wi][0]) = h[1];
            *reinterpret_cast<half8 *>(&wl_s[buf][0][wi][0]) = l[0];
            *reinterpret_cast<half8 *>(&wl_s[buf][1][wi][0]) = l[1];
        }
    };
    auto load_a = [&](int s, half8 &ah, half8 &al) {
        const size_t o = ((size_t)tile * ksteps + s) * 64 + lane;
        ah = reinterpret_cast<const half8 *>(wh)[o];
        al = reinterpret_cast<const half8 *>(wl)[o];
    };
    f32x16 acc[PT];
#pragma unroll
    for (int t = 0; t < PT; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
    float wv[NP][16];
    load_win(0, wv);
    store_win(0, wv);
    half8 ah, al;
    load_a(0, ah, al);
    __syncthreads();
    const int nsteps = ncb * ks;  // the steps past these (stage padding) hold zero weights
    for (int cb = 0; cb < ncb; cb++) {
        const int buf = cb & 1;
        const bool more = cb + 1 < ncb;  // uniform
        if (more) load_win(cb + 1, wv);
        for (int tap = 0; tap < ks; tap++) {
            const int s = cb * ks + tap;
            half8 nh, nl;
            load_a(s + 1 < nsteps ? s + 1 : s, nh, nl);
#pragma unroll
            for (int t = 0; t < PT; t++) {
                const int p = t * 32 + col + tap * dil;
                const half8 bh = *reinterpret_cast<const half8 *>(&wh_s[buf][half][p][0]);
                const half8 bl = *reinterpret_cast<const half8 *>(&wl_s[buf][half][p][0]);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, acc[t], 0, 0, 0);
            }
            ah = nh;
            al = nl;
        }
        // buf ^ 1 was last read in channel block cb - 1, before the last barrier
        if (more) store_win(buf ^ 1, wv);
        __syncthreads();
    }
    // D layout: lane l, register r -> row (r / 4) * 8 + (l / 32) * 4 + r % 4,
    // column l % 32
    const int sc = -(ex + P.ew);
#pragma unroll
    for (int t = 0; t < PT; t++) {
        const int n = n0 + t * 32 + col;
        if (n >= len) continue;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = 32 * tile + (r >> 2) * 8 + half * 4 + (r & 3);
            if (m >= P.M) continue;
            float v = ldexpf(acc[t][r], sc);
            if (P.bias) v += P.bias[m];
            if (P.act == DEC_ACT_GELU) v = dec_gelu(v);
            float *dst = P.c + (long long)m * P.ldc + (long long)n * P.out_stride + phase;
            switch (P.epi) {
                case DEC_EPI_STORE: *dst = v; break;
                case DEC_EPI_ACCUM: *dst += v; break;
                case DEC_EPI_SCALED_RESID: *dst += P.scale[m] * v; break;
                case DEC_EPI_RESID_IN: *dst = P.resid[dst - P.c] + (P.scale ? P.scale[m] * v : v); break;
                default: *dst = v < -1.0f ? -1.0f : (v > 1.0f ? 1.0f : v); break;  // DEC_EPI_CLAMP (NaN stays)
            }
        }
    }
}

unsigned blocks_for(size_t n, unsigned per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

void launch_dec_gather(hipStream_t st, const DecGatherParams &p, int frames) {
    hipLaunchKernelGGL(k_dec_gather, dim3((unsigned)frames), dim3(256), 0, st, p);
}

void launch_dec_rmsnorm(hipStream_t st, const float *x, const float *gamma, int rows, int n, float eps, float *out) {
    hipLaunchKernelGGL(k_dec_rmsnorm, dim3((unsigned)rows), dim3(256), 0, st, x, gamma, n, eps, out);
}

void launch_dec_rope(hipStream_t st, float *q, float *k, int T, int heads, int hd, const float *cs, const float *sn,
                     int rows, int ld) {
    const size_t n = (size_t)T * heads * (hd / 2);
    hipLaunchKernelGGL(k_dec_rope, dim3(blocks_for(n, 256)), dim3(256), 0, st, q, k, T, heads, hd, cs, sn, rows, ld);
}

void launch_dec_attn(hipStream_t st, const DecAttnParams &p) {
    hipLaunchKernelGGL(k_dec_attn, dim3(blocks_for((size_t)p.T * p.heads, 4)), dim3(256), 0, st, p);
}

void launch_dec_swiglu(hipStream_t st, const float *g, const float *u, int rows, int width, int ld, float *out) {
    const size_t n = (size_t)rows * width;
    hipLaunchKernelGGL(k_dec_swiglu, dim3(blocks_for(n, 256)), dim3(256), 0, st, g, u, rows, width, ld, out);
}

void launch_dec_dwconv(hipStream_t st, const float *x, const float *w, const float *b, int ch, int len, int ks,
                       float *out) {
    hipLaunchKernelGGL(k_dec_dwconv, dim3(blocks_for((size_t)ch * len, 256)), dim3(256), 0, st, x, w, b, ch, len, ks,
                       out);
}

void launch_dec_lnorm(hipStream_t st, const float *x, const float *g, const float *b, int ch, int len, float eps,
                      float *out) {
    // the tiled kernel while its [ch][TS] tile fits 64 KiB of LDS
    const size_t lds16 = (size_t)ch * 16 * sizeof(float), lds8 = (size_t)ch * 8 * sizeof(float);
    if (lds16 <= 65536)
        hipLaunchKernelGGL(k_dec_lnorm_tile<16>, dim3((unsigned)((len + 15) / 16)), dim3(256), lds16, st, x, g, b, ch,
                           len, eps, out);
    else if (lds8 <= 65536)
        hipLaunchKernelGGL(k_dec_lnorm_tile<8>, dim3((unsigned)((len + 7) / 8)), dim3(256), lds8, st, x, g, b, ch, len,
                           eps, out);
    else
        hipLaunchKernelGGL(k_dec_lnorm, dim3(blocks_for((size_t)len, 64)), dim3(64), 0, st, x, g, b, ch, len, eps, out);
}

void launch_dec_snake(hipStream_t st, const float *x, const float *alpha, const float *beta, int ch, int len,
                      float *out, unsigned *amax, const float *add, float *sum) {
    // about kSnakeBlocks blocks in all, at least one per channel (rows of a
    // multiple of 4 samples take 4 per thread and iteration)
    const size_t items = (len & 3) == 0 ? (size_t)len / 4 : (size_t)len;
    const unsigned per_row = std::max(1u, std::min<unsigned>(blocks_for(items, 256), kSnakeBlocks / (unsigned)ch));
    hipLaunchKernelGGL(k_dec_snake, dim3(per_row, (unsigned)ch), dim3(256), 0, st, x, alpha, beta, ch, len, out, amax,
                       add, sum);
}

void launch_dec_fill_u32(hipStream_t st, unsigned *p, int n, unsigned v) {
    hipLaunchKernelGGL(k_dec_fill_u32, dim3(blocks_for((size_t)n, 256)), dim3(256), 0, st, p, n, v);
}

void launch_dec_conv_repack(hipStream_t st, const float *w, long long sm, long long sci, int k0, int kd, int M, int cin,
                            int taps, int cin16, int mtiles, int ksteps, int ew, _Float16 *wh, _Float16 *wl) {
    const size_t n = (size_t)mtiles * ksteps * 64;
    hipLaunchKernelGGL(k_dec_conv_repack, dim3(blocks_for(n, 256)), dim3(256), 0, st, w, sm, sci, k0, kd, M, cin,
                       taps, cin16, mtiles, ksteps, ew, wh, wl);
}

template <bool KF>
static void launch_conv_mfma_kf(hipStream_t st, const DecConvMfmaParams &p, int mt) {
    const dim3 grid(blocks_for((size_t)p.len, 128), (unsigned)(p.mtiles / mt), (unsigned)std::max(1, p.nphase));
    switch (mt) {
        case 4: hipLaunchKernelGGL((k_dec_conv_mfma<4, KF>), grid, dim3(256), 0, st, p); break;
        case 3: hipLaunchKernelGGL((k_dec_conv_mfma<3, KF>), grid, dim3(256), 0, st, p); break;
        case 2: hipLaunchKernelGGL((k_dec_conv_mfma<2, KF>), grid, dim3(256), 0, st, p); break;
        default: hipLaunchKernelGGL((k_dec_conv_mfma<1, KF>), grid, dim3(256), 0, st, p); break;
    }
}

// MT: the largest of 4, 3, 2, 1 that divides the tile count (a block's
// tiles share each gathered B operand); a launch that would leave CUs idle
// even at MT = 1 (fewer than kDecFillBlocks blocks) splits K over the
// block's waves instead (k_dec_conv_mfma_ks); channel-first convolutions of
// 3 or more taps take k_dec_conv_win.  QTTS_DEC_CONV=tiles or =split forces
// the long-decode kernels (MT by divisibility alone) or the K split for
// every launch, so that short decodes can check both against a reference.
void launch_dec_conv_mfma(hipStream_t st, const DecConvMfmaParams &p) {
    const char *plan = std::getenv("QTTS_DEC_CONV");
    const bool force_tiles = plan && std::strcmp(plan, "tiles") == 0, force_split = plan && std::strcmp(plan, "split") == 0;
    const bool kf = p.sxc == 1 && p.cin % 8 == 0 && p.sxn % 4 == 0 && ((uintptr_t)p.x & 15) == 0;
    const size_t nph = (size_t)std::max(1, p.nphase);  // a transposed convolution's phases in one launch
    if (force_split ||
        (!force_tiles && (size_t)blocks_for((size_t)p.len, 128) * (size_t)p.mtiles * nph < kDecFillBlocks)) {
        const dim3 grid(blocks_for((size_t)p.len, 32), (unsigned)p.mtiles, (unsigned)nph);
        if (kf)
            hipLaunchKernelGGL(k_dec_conv_mfma_ks<true>, grid, dim3(256), 0, st, p);
        else
            hipLaunchKernelGGL(k_dec_conv_mfma_ks<false>, grid, dim3(256), 0, st, p);
        return;
    }
    int mt = p.mtiles % 4 == 0 ? 4 : p.mtiles % 3 == 0 ? 3 : p.mtiles % 2 == 0 ? 2 : 1;
    if (!force_tiles && (size_t)blocks_for((size_t)p.len, 128) * (size_t)(p.mtiles / mt) * nph < 256) mt = 1;
    if (p.ksize >= 3 && p.sxn == 1 && p.sxc == p.len && 128 + (p.ksize - 1) * p.dilation <= 256) {
        // a channel-first convolution with 3 or more taps whose window fits the block's threads
        const dim3 grid(blocks_for((size_t)p.len, 128), (unsigned)(p.mtiles / mt), (unsigned)nph);
        switch (mt) {
            case 4: hipLaunchKernelGGL(k_dec_conv_win_tw<4>, grid, dim3(256), 0, st, p); break;
            case 3: hipLaunchKernelGGL(k_dec_conv_win_tw<3>, grid, dim3(192), 0, st, p); break;
            case 2: hipLaunchKernelGGL(k_dec_conv_win<2>, grid, dim3(256), 0, st, p); break;
            default: hipLaunchKernelGGL(k_dec_conv_win<1>, grid, dim3(256), 0, st, p); break;
        }
        return;
    }
    if (kf)
        launch_conv_mfma_kf<true>(st, p, mt);
    else
        launch_conv_mfma_kf<false>(st, p, mt);
}

void launch_dec_absmax(hipStream_t st, const float *x, size_t n, unsigned *amax) {
    // at most 512 blocks: each folds its maximum into one of the 64 slots
    // with one atomic, so fewer blocks queue fewer atomics per slot
    const unsigned blocks = std::min<unsigned>(blocks_for((n + 3) / 4, 256), 512u);
    hipLaunchKernelGGL(k_dec_absmax, dim3(blocks), dim3(256), 0, st, x, n, amax);
}

}  // namespace qtts
