// device_common.h — small device helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "internal.h"

namespace qtts {

// Global-address-space view of a pointer.  Pointers read out of structs in
// memory are generic to the compiler, and generic (flat) accesses count
// against both vmcnt and lgkmcnt: every later LDS or scalar-load wait would
// then also wait for outstanding HBM loads.  Accesses through glb() are
// global_load/global_store.
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T *glb(T *p) {
    return (__attribute__((address_space(1))) T *)p;
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// Read-only (constant address space) view, for op descriptors: loads through
// it are scalar loads (lgkmcnt), which do not wait behind outstanding vector
// loads the way a vector load of a descriptor field would (vmcnt retires in
// order).
#define KCONST __attribute__((address_space(4)))

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Lane exchange within rows of 16 lanes through DPP (a VALU operand
// modifier: no LDS round trip, unlike __shfl_xor's ds_bpermute).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- 7-i within each 8
constexpr int kDppMirror = 0x140;      // lane i <- 15-i within each 16
constexpr int kDppRowShl4 = 0x104;     // lane i <- i+4 within each 16
constexpr int kDppRowShl8 = 0x108;     // lane i <- i+8
constexpr int kDppRowShr4 = 0x114;     // lane i <- i-4
constexpr int kDppRowShr8 = 0x118;     // lane i <- i-8

// dpp<A>(v) on lanes where `pick`, dpp<B>(v) elsewhere.  Both are computed
// by every lane: a DPP read from a lane that is inactive (as it would be if
// the compiler turned the choice into a branch) returns nothing.
template <int A, int B>
__device__ __forceinline__ float dpp_pick(bool pick, float v) {
    float ra = dpp<A>(v), rb = dpp<B>(v);
    asm volatile("" : "+v"(ra), "+v"(rb));
    return pick ? ra : rb;
}

// Sum over each row of 16 lanes; every lane of the row gets it.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppMirror>(v));
    return v;
}
__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// v[l] + v[l ^ 32] on every lane (v_permlane32_swap).
__device__ __forceinline__ float halves_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum / max over the 64-lane wave; every lane gets the result.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = row16_max(v);
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Cross-workgroup traffic inside one kernel goes through agent-scope atomic
// loads/stores, which the gfx950 memory model performs at the device
// coherence point (sc1).  That orders a handoff without an agent-scope
// fence, whose L2 writeback + invalidate per workgroup costs more than a
// small GEMV.
__device__ __forceinline__ void st_dev(float *p, float v) {
    __hip_atomic_store(glb(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float *p) {
    return __hip_atomic_load(glb(const_cast<float *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u32(uint32_t *p, uint32_t v) {
    __hip_atomic_store(glb(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev_u32(const uint32_t *p) {
    return __hip_atomic_load(glb(const_cast<uint32_t *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_dev_i32(const int *p) {
    return __hip_atomic_load(glb(const_cast<int *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_i32(int *p, int v) {
    __hip_atomic_store(glb(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev_u64(const uint64_t *p) {
    return __hip_atomic_load(glb(const_cast<uint64_t *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u64(uint64_t *p, uint64_t v) {
    __hip_atomic_store(glb(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Counts one arrival; returns the count before the increment.
__device__ __forceinline__ unsigned arrive_dev(unsigned *ctr) {
    return __hip_atomic_fetch_add(glb(ctr), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void reset_dev(unsigned *ctr) {
    __hip_atomic_store(glb(ctr), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until this wave's earlier memory operations have completed.
// Waits until every memory operation this wave issued has completed (its
// stores acknowledged), so a later store that other blocks poll is ordered
// after them.  (A workgroup-scope release fence emits no wait on gfx950.)
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// xorshift64 (13, 7, 17) and (state as f32) / (u64::MAX as f32), both
// conversions rounding to nearest (src/generate_new.rs:17-22).
__device__ __forceinline__ float simple_rand_dev(uint64_t *state) {
    uint64_t s = *state;
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    *state = s;
    return (float)s / 18446744073709551616.0f;
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Dwords per row of a panel slice of C columns (C = 4: 16 bits in dword 0).
template <int C>
constexpr int q4_slice_dwords() {
    return C >= 8 ? C / 8 : 1;
}

// One row of a C-column slice (`row` points at the slice's bytes inside a
// 16-byte panel row), loaded with one non-temporal load of C / 2 bytes.
template <int C>
__device__ __forceinline__ void q4_slice_load(const uint8_t *row, uint32_t (&wd)[q4_slice_dwords<C>()]) {
    if constexpr (C == 32) {
        const u32x4 v = __builtin_nontemporal_load(glb(reinterpret_cast<const u32x4 *>(row)));
        wd[0] = v.x;
        wd[1] = v.y;
        wd[2] = v.z;
        wd[3] = v.w;
    } else if constexpr (C == 16) {
        const u32x2 v = __builtin_nontemporal_load(glb(reinterpret_cast<const u32x2 *>(row)));
        wd[0] = v.x;
        wd[1] = v.y;
    } else if constexpr (C == 8) {
        wd[0] = __builtin_nontemporal_load(glb(reinterpret_cast<const uint32_t *>(row)));
    } else {
        wd[0] = __builtin_nontemporal_load(glb(reinterpret_cast<const uint16_t *>(row)));
    }
}

// acc[m][c] += sx[m] * nib_c over one row of a C-column slice (nibble c at
// bits 4 * (c % 8) of dword c / 8; the caller subtracts 8 * sum(sx) per
// column once), given sa = sx * 2^24 and sb = sx * 2^20, both exact.  Two
// nibbles at a time are masked into the halves of a register, where they
// read as f16 denormals: n * 2^-24 from bits 0-3 of a half, n * 2^-20 from
// bits 4-7.  v_fma_mix_f32 converts a half exactly, so every term is
// sx * n rounded once, the same sums as fmaf(sx, (float)n, acc), in 13 VALU
// operations per 8 nibbles (a shift, 4 masks, 8 FMAs).
template <int M, int C>
__device__ __forceinline__ void q4_mix_row(const uint32_t (&wd)[q4_slice_dwords<C>()], const float (&sa)[M],
                                           const float (&sb)[M], float (&acc)[M][C]) {
#pragma unroll
    for (int d = 0; d < q4_slice_dwords<C>(); d++) {
        const uint32_t w = wd[d], w8 = w >> 8;
        const f16x2 h0 = __builtin_bit_cast(f16x2, w & 0x000F000Fu);   // nibbles 0, 4
        const f16x2 h1 = __builtin_bit_cast(f16x2, w & 0x00F000F0u);   // nibbles 1, 5
        const f16x2 h2 = __builtin_bit_cast(f16x2, w8 & 0x000F000Fu);  // nibbles 2, 6
        const f16x2 h3 = __builtin_bit_cast(f16x2, w8 & 0x00F000F0u);  // nibbles 3, 7
#pragma unroll
        for (int m = 0; m < M; m++) {
            float *a = &acc[m][8 * d];
            a[0] = fmaf(sa[m], (float)h0.x, a[0]);
            a[1] = fmaf(sb[m], (float)h1.x, a[1]);
            a[2] = fmaf(sa[m], (float)h2.x, a[2]);
            a[3] = fmaf(sb[m], (float)h3.x, a[3]);
            if constexpr (C >= 8) {
                a[4] = fmaf(sa[m], (float)h0.y, a[4]);
                a[5] = fmaf(sb[m], (float)h1.y, a[5]);
                a[6] = fmaf(sa[m], (float)h2.y, a[6]);
                a[7] = fmaf(sb[m], (float)h3.y, a[7]);
            }
        }
    }
}

// Lane exchange of DPP stage S (partner lane = lane ^ (1 << S)) within rows
// of 16 lanes; `bit` is this lane's bit S.
template <int S>
__device__ __forceinline__ float dpp_xchg(bool bit, float v) {
    if constexpr (S == 0) return dpp<kDppXor1>(v);
    else if constexpr (S == 1) return dpp<kDppXor2>(v);
    else if constexpr (S == 2) return dpp_pick<kDppRowShr4, kDppRowShl4>(bit, v);
    else return dpp_pick<kDppRowShr8, kDppRowShl8>(bit, v);
}

// One stage over the N values v[0..N): with N > 1 the set is halved (lanes
// with `bit` keep the upper half and receive the partner's copy of it),
// otherwise the partner's value is added.
template <int N, int S, int C>
__device__ __forceinline__ void dpp_stage(float (&v)[C], bool bit) {
    if constexpr (N > 1) {
#pragma unroll
        for (int j = 0; j < N / 2; j++) {
            const float keep = bit ? v[j + N / 2] : v[j], send = bit ? v[j] : v[j + N / 2];
            v[j] = keep + dpp_xchg<S>(bit, send);
        }
    } else {
        v[0] += dpp_xchg<S>(bit, v[0]);
    }
}

// v summed over the four 16-lane rows of the wave, on every lane (for its
// position in the row): rows (0 + 1) and (2 + 3) by v_permlane16_swap, then
// the two halves by v_permlane32_swap.
__device__ __forceinline__ float rows4_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Column sums of a 256-thread block's acc[C] (C = 32, 16, 8 or 4), step
// one: four DPP stages within each row of 16 lanes leave every lane with
// max(C / 16, 1) column sums over its row, the rows of a wave are added by
// lane swaps, and lanes 0-15 store the wave's sums to red[wave][C] (lanes
// holding the same column store the same value).  After a barrier,
// red[0..3][c] summed over the waves is column c.
template <int C>
__device__ __forceinline__ void dpp_reduce(const float (&acc)[C], float *red) {
    const int tid = threadIdx.x, r16 = tid & 15, wave = tid >> 6;
    const bool b0 = r16 & 1, b1 = r16 & 2, b2 = r16 & 4, b3 = r16 & 8;
    float v[C];
#pragma unroll
    for (int j = 0; j < C; j++) v[j] = acc[j];
    dpp_stage<C, 0>(v, b0);
    dpp_stage<(C / 2 > 1 ? C / 2 : 1), 1>(v, b1);
    dpp_stage<(C / 4 > 1 ? C / 4 : 1), 2>(v, b2);
    dpp_stage<(C / 8 > 1 ? C / 8 : 1), 3>(v, b3);
    constexpr int NV = C / 16 > 1 ? C / 16 : 1;
#pragma unroll
    for (int j = 0; j < NV; j++) v[j] = rows4_sum(v[j]);
    const int col = (b0 ? C / 2 : 0) + (b1 ? C / 4 : 0) + (C >= 8 && b2 ? C / 8 : 0) + (C >= 16 && b3 ? C / 16 : 0);
    if ((tid & 63) < 16) {
#pragma unroll
        for (int j = 0; j < NV; j++) red[wave * C + col + j] = v[j];
    }
}

constexpr int kDppRowRor8 = 0x128;  // lane i <- (i + 8) mod 16: the partner i ^ 8 within each 16

// Column sums of a block's acc[32] (one partial per column per lane), step
// one: halving stages leave each lane with one column's sum over the 64 lanes
// of its wave.  Lane bit 5 goes first, by v_permlane32_swap (the upper half
// of one register swapped with the lower half of another: one swap and one
// add per pair of columns), then bit 4 by v_permlane16_swap, bits 0-2 by DPP
// within rows of 16 lanes, and bit 3 as a plain add of the value rotated by 8
// in the row, so lanes l and l ^ 8 end with the same sum.  Lanes with bit 3
// clear store it to red[wave * 32 + col].  After a barrier, red[w][c] summed
// over the waves is column c.
__device__ __forceinline__ void lane_reduce32(const float (&acc)[32], float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; j++) v[j] = acc[j];
    // bit 5: lanes < 32 keep columns 0..15, lanes >= 32 columns 16..31
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[j + 16]), false, false);
        v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    // bit 4: rows 0 and 2 keep the first 8 of their 16, rows 1 and 3 the last 8
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[j]), __float_as_uint(v[j + 8]), false, false);
        v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const bool b0 = lane & 1, b1 = lane & 2, b2 = lane & 4, b3 = lane & 8;
    dpp_stage<8, 0>(v, b0);
    dpp_stage<4, 1>(v, b1);
    dpp_stage<2, 2>(v, b2);
    v[0] += dpp<kDppRowRor8>(v[0]);
    const int col = ((lane & 32) ? 16 : 0) + ((lane & 16) ? 8 : 0) + (b0 ? 4 : 0) + (b1 ? 2 : 0) + (b2 ? 1 : 0);
    if (!b3) red[wave * 32 + col] = v[0];
}

// The same for acc[16] (half-panel tasks): bits 5 and 4 by lane swaps, bits
// 0 and 1 by DPP halving, bits 2 and 3 as plain adds, so lanes that differ in
// bits 2 and 3 hold the same column sum; lanes with both clear store it to
// red[wave * 16 + col].
__device__ __forceinline__ void lane_reduce16(const float (&acc)[16], float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; j++) v[j] = acc[j];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[j + 8]), false, false);
        v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[j]), __float_as_uint(v[j + 4]), false, false);
        v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const bool b0 = lane & 1, b1 = lane & 2, b2 = lane & 4;
    dpp_stage<4, 0>(v, b0);
    dpp_stage<2, 1>(v, b1);
    v[0] += dpp_xchg<2>(b2, v[0]);
    v[0] += dpp<kDppRowRor8>(v[0]);
    const int col = ((lane & 32) ? 8 : 0) + ((lane & 16) ? 4 : 0) + (b0 ? 2 : 0) + (b1 ? 1 : 0);
    if ((lane & 12) == 0) red[wave * 16 + col] = v[0];
}

// f32 sum of s[0..n) in index order by one thread (the order the reference
// sums in).  The LDS reads are issued 32 at a time so the add chain, not the
// read latency, sets the pace.  s is 16-byte aligned.
__device__ __forceinline__ float seq_sum(const float *s, int n) {
    float sum = 0.0f;
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        float4 v[8];
#pragma unroll
        for (int q = 0; q < 8; q++) v[q] = *reinterpret_cast<const float4 *>(&s[i + 4 * q]);
#pragma unroll
        for (int q = 0; q < 8; q++) {
            sum += v[q].x;
            sum += v[q].y;
            sum += v[q].z;
            sum += v[q].w;
        }
    }
    for (; i < n; i++) sum += s[i];
    return sum;
}

// out[i] = element (row, col0 + i * stride) of a panel-major Q4 weight for
// columns < ncol, else 0 (row < w.K).  All loads are issued before any is
// used, as in embed_lookup_q4 (src/gemv.rs:377-400) per element.
template <int N, typename Q4>
__device__ __forceinline__ void q4_gather(const Q4 &w, uint32_t row, int col0, int stride, int ncol, float (&out)[N]) {
    uint32_t by[N], sc[N];
#pragma unroll
    for (int i = 0; i < N; i++) {
        const int col = min(col0 + i * stride, ncol - 1);
        const size_t r = (size_t)(col >> 5) * w.K + row;
        by[i] = glb(reinterpret_cast<const uint8_t *>(w.wq))[r * 16 + ((col & 31) >> 1)];
        sc[i] = glb(w.ws)[r];
    }
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" : "+v"(by[i]), "+v"(sc[i]));
#pragma unroll
    for (int i = 0; i < N; i++) {
        const int col = col0 + i * stride;
        const int nib = (col & 1) ? (int)(by[i] >> 4) : (int)(by[i] & 15u);
        out[i] = col < ncol ? f16_to_f32((uint16_t)sc[i]) * (float)(nib - 8) : 0.0f;
    }
}

// Element (row, col) of a panel-major Q4 weight: f32(scale) * (nib - 8),
// the product embed_lookup_q4 forms (src/gemv.rs:388-396); exact.
template <typename Q4>
__device__ __forceinline__ float q4_element(const Q4 &w, uint32_t row, int col) {
    const size_t r = (size_t)(col >> 5) * w.K + row;
    const uint8_t byte = glb(reinterpret_cast<const uint8_t *>(w.wq))[r * 16 + ((col & 31) >> 1)];
    const int nib = (col & 1) ? (byte >> 4) : (byte & 15);
    return f16_to_f32(glb(w.ws)[r]) * (float)(nib - 8);
}

}  // namespace qtts
