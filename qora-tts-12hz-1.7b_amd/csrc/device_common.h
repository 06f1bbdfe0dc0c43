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
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup"); }

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

// acc[m][c] += sx[m] * nib_c for the 32 nibbles of one panel row (nib_c in
// 0..15; the caller subtracts 8 * sum(sx) per column once).  The nibbles are
// split into bytes so each converts with one v_cvt_f32_ubyteN.
template <int M>
__device__ __forceinline__ void q4_fma_row(const u32x4 w, const float (&sx)[M], float (&acc)[M][32]) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int d = 0; d < 4; d++) {
        uint32_t lo = wd[d] & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6
        uint32_t hi = (wd[d] >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
        // opaque to the compiler, which would otherwise fold the byte
        // conversions back into per-nibble bit-field extracts
        asm volatile("" : "+v"(lo), "+v"(hi));
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float q0 = (float)((lo >> (8 * b)) & 0xFFu), q1 = (float)((hi >> (8 * b)) & 0xFFu);
#pragma unroll
            for (int m = 0; m < M; m++) {
                acc[m][d * 8 + 2 * b] = fmaf(sx[m], q0, acc[m][d * 8 + 2 * b]);
                acc[m][d * 8 + 2 * b + 1] = fmaf(sx[m], q1, acc[m][d * 8 + 2 * b + 1]);
            }
        }
    }
}

// Column sums of a 256-thread block's acc[32], step one: four DPP exchange
// stages within each row of 16 lanes halve the column set per stage (lane
// bit s keeps the lower or upper half and receives the partner's copy of
// it), leaving each lane two column sums over its row, stored to
// red[row][32] (row = tid / 16).  After a barrier, red[0..15][c] summed over
// the rows is column c.
__device__ __forceinline__ void dpp_reduce32(const float (&acc)[32], float *red) {
    const int tid = threadIdx.x, r16 = tid & 15, row = tid >> 4;
    const bool b0 = r16 & 1, b1 = r16 & 2, b2 = r16 & 4, b3 = r16 & 8;
    const int colbase = (b0 ? 16 : 0) + (b1 ? 8 : 0) + (b2 ? 4 : 0) + (b3 ? 2 : 0);
    float v16[16], v8[8], v4[4], v2[2];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const float keep = b0 ? acc[j + 16] : acc[j], send = b0 ? acc[j] : acc[j + 16];
        v16[j] = keep + dpp<kDppXor1>(send);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const float keep = b1 ? v16[j + 8] : v16[j], send = b1 ? v16[j] : v16[j + 8];
        v8[j] = keep + dpp<kDppXor2>(send);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float keep = b2 ? v8[j + 4] : v8[j], send = b2 ? v8[j] : v8[j + 4];
        v4[j] = keep + dpp_pick<kDppRowShr4, kDppRowShl4>(b2, send);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const float keep = b3 ? v4[j + 2] : v4[j], send = b3 ? v4[j] : v4[j + 2];
        v2[j] = keep + dpp_pick<kDppRowShr8, kDppRowShl8>(b3, send);
    }
    red[row * 32 + colbase] = v2[0];
    red[row * 32 + colbase + 1] = v2[1];
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
