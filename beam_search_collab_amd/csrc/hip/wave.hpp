// Wave64 building blocks for gfx950 (CDNA4): lane exchanges, ballots, wave-scope sync.
//
// Exchanges used by the reductions and the bitonic sorter:
//   xor 1, 2      DPP quad_perm                      (VALU, no LDS traffic)
//   xor 4, 8      two DPP mirrors (row_half_mirror/row_mirror composed with quad reverse)
//   xor 16        v_permlane16_swap + a select       (VALU)
//   xor 32        v_permlane32_swap + a select       (VALU)
//   shift by one  ds_bpermute
// Butterfly reductions need less once the lanes of each group agree: one DPP mirror for the
// partner quad or half-row, and the two results of one lane swap combined without a select
// (partner, group_sum).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bsw {

__device__ __forceinline__ uint32_t lane_id() {
    return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// this lane's bit of a wave-uniform mask (the mask itself becomes the lane condition: no
// vector instruction)
__device__ __forceinline__ bool lane_in(uint64_t m) { return __builtin_amdgcn_inverse_ballot_w64(m); }

// number of set bits of m below this lane
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

__device__ __forceinline__ uint32_t readlane(uint32_t v, uint32_t l) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), static_cast<int>(l)));
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, uint32_t l) {
    const uint32_t lo = readlane(static_cast<uint32_t>(v), l);
    const uint32_t hi = readlane(static_cast<uint32_t>(v >> 32), l);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint32_t uniform(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
    return (static_cast<uint64_t>(uniform(static_cast<uint32_t>(v >> 32))) << 32) | uniform(static_cast<uint32_t>(v));
}

// Orders LDS traffic of the wave: every lane's earlier LDS writes are visible to every
// lane's later LDS reads, and the compiler may not move LDS accesses across it.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// DPP controls (GFX9 encoding)
constexpr int DPP_QP_XOR1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int DPP_QP_XOR2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int DPP_QP_XOR3 = 0x1B;   // quad_perm [3,2,1,0]
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i -> 7-i within 8
constexpr int DPP_MIRROR = 0x140;       // lane i -> 15-i within 16

template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// value of lane (this lane ^ S)
template <int S>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    if constexpr (S == 1) {
        return dpp<DPP_QP_XOR1>(v);
    } else if constexpr (S == 2) {
        return dpp<DPP_QP_XOR2>(v);
    } else if constexpr (S == 4) {
        return dpp<DPP_QP_XOR3>(dpp<DPP_HALF_MIRROR>(v));  // (i ^ 7) ^ 3 = i ^ 4
    } else if constexpr (S == 8) {
        return dpp<DPP_HALF_MIRROR>(dpp<DPP_MIRROR>(v));   // (i ^ 15) ^ 7 = i ^ 8
    } else if constexpr (S == 16) {
        // v_permlane16_swap (gfx950): of swap(v, v), result 0 holds rows 0,0,2,2 and result 1
        // rows 1,1,3,3 of v (rows of 16 lanes), so rows 0 and 2 take result 1
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return lane_in(0x0000FFFF0000FFFFull) ? r[1] : r[0];
    } else {
        static_assert(S == 32, "xor distance must be a power of two below 64");
        // v_permlane32_swap (gfx950): of swap(v, v), result 0 holds the lower half of v twice
        // and result 1 the upper half twice, so lanes 0-31 take result 1
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return lane_in(0x00000000FFFFFFFFull) ? r[1] : r[0];
    }
}

template <int S>
__device__ __forceinline__ float xor_lane_f(float v) {
    return __uint_as_float(xor_lane<S>(__float_as_uint(v)));
}
template <int S>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v) {
    const uint32_t lo = xor_lane<S>(static_cast<uint32_t>(v));
    const uint32_t hi = xor_lane<S>(static_cast<uint32_t>(v >> 32));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// run-time distance (folded when the call is unrolled with a constant s)
__device__ __forceinline__ uint64_t xor_lane64_rt(uint64_t v, uint32_t s) {
    switch (s) {
    case 1: return xor_lane64<1>(v);
    case 2: return xor_lane64<2>(v);
    case 4: return xor_lane64<4>(v);
    case 8: return xor_lane64<8>(v);
    case 16: return xor_lane64<16>(v);
    default: return xor_lane64<32>(v);
    }
}

// Exchanges of a butterfly reduction.  Once every aligned group of S lanes holds one value
// (the reduction's earlier steps made it so), any lane of the partner group will do: at
// distances 4 and 8 one DPP mirror reaches the other quad / half-row (xor_lane needs two),
// and at 16 and 32 one lane swap leaves the pair's two values in the two results in every
// lane, so no select is needed (op(r[0], r[1]) is the pair's result).  The results are the
// xor butterfly's bit for bit as long as op is commutative.
template <int S>
__device__ __forceinline__ uint32_t partner(uint32_t v) {
    static_assert(S == 4 || S == 8, "mirror partners exist at distances 4 and 8");
    return S == 4 ? dpp<DPP_HALF_MIRROR>(v) : dpp<DPP_MIRROR>(v);
}
template <int S>
__device__ __forceinline__ float partner_f(float v) {
    return __uint_as_float(partner<S>(__float_as_uint(v)));
}

// Load of a T at byte offset `off` from a wave-uniform base (a record whose address the
// wave computed from a picked node).  The empty asm (it emits nothing) keeps the compiler
// from hoisting the offset's 64-bit extension out of the caller's loop, so the load takes
// the base from scalar registers and the 32-bit offset from a vector register
// (global_load ... voffset, saddr): no 64-bit address arithmetic per lane and load.
template <typename T>
__device__ __forceinline__ T load_off(const void* base, uint32_t off) {
    asm volatile("" : "+v"(off));
    return *reinterpret_cast<const T*>(static_cast<const char*>(base) + off);
}

// value of lane (this lane - 1); lane 0 gets lane 63's value
__device__ __forceinline__ uint32_t prev_lane(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_ds_bpermute(static_cast<int>(((lane_id() + 63u) & 63u) << 2), static_cast<int>(v)));
}

// Sum over aligned groups of G lanes (G a power of two <= 64) by an xor butterfly:
// p_l += p_{l^s} for s = 1, 2, ..., G/2, the partners from 4 on taken by the reduction
// exchanges above.  Every lane of a group ends with the same value (float addition is
// commutative).  All 64 lanes must be active.
__device__ __forceinline__ float group_sum(float p, uint32_t G) {
    if (G > 1) p = p + xor_lane_f<1>(p);
    if (G > 2) p = p + xor_lane_f<2>(p);
    if (G > 4) p = p + partner_f<4>(p);
    if (G > 8) p = p + partner_f<8>(p);
    if (G > 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(p), __float_as_uint(p), false, false);
        p = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    if (G > 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(p), __float_as_uint(p), false, false);
        p = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    return p;
}

__device__ __forceinline__ uint32_t group_sum_u32(uint32_t p, uint32_t G) {
    if (G > 1) p += xor_lane<1>(p);
    if (G > 2) p += xor_lane<2>(p);
    if (G > 4) p += partner<4>(p);
    if (G > 8) p += partner<8>(p);
    if (G > 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(p, p, false, false);
        p = r[0] + r[1];
    }
    if (G > 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(p, p, false, false);
        p = r[0] + r[1];
    }
    return p;
}

__device__ __forceinline__ float wave_min(float v) {
    v = fminf(v, xor_lane_f<1>(v));
    v = fminf(v, xor_lane_f<2>(v));
    v = fminf(v, xor_lane_f<4>(v));
    v = fminf(v, xor_lane_f<8>(v));
    v = fminf(v, xor_lane_f<16>(v));
    v = fminf(v, xor_lane_f<32>(v));
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, xor_lane_f<1>(v));
    v = fmaxf(v, xor_lane_f<2>(v));
    v = fmaxf(v, xor_lane_f<4>(v));
    v = fmaxf(v, xor_lane_f<8>(v));
    v = fmaxf(v, xor_lane_f<16>(v));
    v = fmaxf(v, xor_lane_f<32>(v));
    return v;
}

}  // namespace bsw
