// Cross-lane primitives for gfx950's 64-lane wavefronts, built on DPP row
// shifts (a VALU operand modifier: no LDS round trip), the CDNA4 permlane
// swaps for the steps that cross a 16-lane row, and readlane for wave-wide
// results.  ds_bpermute (what __shfl_* lowers to) goes through the LDS
// crossbar and costs an LDS round trip per step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace swann {

// The value held by lane l + OFF, for lane l of an aligned group of 2*OFF
// lanes whose lower half asks (lanes of the upper half get an unspecified
// value).  OFF <= 8 stays inside a DPP row (row_shl; a lane whose source
// falls off its row reads 0); OFF = 16 and 32 use the row and half-wave swaps.
template <int OFF>
__device__ __forceinline__ float lane_up(float v) {
    static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32,
                  "lane_up: OFF must be a power of two up to 32");
    const unsigned u = __builtin_bit_cast(unsigned, v);
    if constexpr (OFF <= 8) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, (int)u, 0x100 + OFF, 0xF,
                                                                     0xF, true));
    } else {
        // v_permlane16_swap: odd rows (16 lanes) of the first operand trade
        // places with even rows of the second, so afterwards the second holds,
        // in each even row, the first's row above.  v_permlane32_swap does the
        // same for half-waves.  Written as inline assembly with both operands
        // read-write: through the builtin, this compiler (ROCm 7.2, gfx950)
        // was seen to read the first result's register where the second
        // result was asked for.  The s_nops cover the VALU-write -> permlane
        // read hazard on the way in and the permlane write -> VALU read on the
        // way out.
        unsigned hi = u, lo = 0u;
        if constexpr (OFF == 16)
            asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1"
                         : "+v"(hi), "+v"(lo));
        else
            asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1"
                         : "+v"(hi), "+v"(lo));
        return __builtin_bit_cast(float, lo);
    }
}

// Tree fold of a TEAM-lane group (TEAM a power of two, 1..64, groups aligned
// to TEAM lanes): for off = TEAM/2 .. 1, lane l < off takes
// fl(acc_l + acc_{l+off}).  The group's total is in its lane 0; other lanes
// hold partial or unspecified values.
template <int TEAM>
__device__ __forceinline__ float team_fold_add(float acc) {
    if constexpr (TEAM >= 64) acc = acc + lane_up<32>(acc);
    if constexpr (TEAM >= 32) acc = acc + lane_up<16>(acc);
    if constexpr (TEAM >= 16) acc = acc + lane_up<8>(acc);
    if constexpr (TEAM >= 8) acc = acc + lane_up<4>(acc);
    if constexpr (TEAM >= 4) acc = acc + lane_up<2>(acc);
    if constexpr (TEAM >= 2) acc = acc + lane_up<1>(acc);
    return acc;
}

// The same fold for integers (exact in any order): lane_up moves bits only.
template <int TEAM>
__device__ __forceinline__ int team_fold_add_i32(int acc) {
    auto up = [](int v, auto off) {
        return __builtin_bit_cast(int, lane_up<decltype(off)::value>(__builtin_bit_cast(float, v)));
    };
    if constexpr (TEAM >= 64) acc += up(acc, std::integral_constant<int, 32>{});
    if constexpr (TEAM >= 32) acc += up(acc, std::integral_constant<int, 16>{});
    if constexpr (TEAM >= 16) acc += up(acc, std::integral_constant<int, 8>{});
    if constexpr (TEAM >= 8) acc += up(acc, std::integral_constant<int, 4>{});
    if constexpr (TEAM >= 4) acc += up(acc, std::integral_constant<int, 2>{});
    if constexpr (TEAM >= 2) acc += up(acc, std::integral_constant<int, 1>{});
    return acc;
}

__device__ __forceinline__ uint64_t umin64(uint64_t a, uint64_t b) { return a < b ? a : b; }

// The value of lane l - OFF within a 16-lane row, or `v` itself where that
// falls off the row (so a running minimum is unchanged there).
template <int OFF>
__device__ __forceinline__ uint64_t row_down64(uint64_t v) {
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    const uint32_t l2 = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, 0x110 + OFF, 0xF, 0xF, false);
    const uint32_t h2 = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, 0x110 + OFF, 0xF, 0xF, false);
    return ((uint64_t)h2 << 32) | l2;
}

// Minimum of v over all 64 lanes (every lane active), returned wave-uniform;
// a lane whose row_shr source falls off its row keeps its own value.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    auto mn = [](uint32_t a, uint32_t b) { return a < b ? a : b; };
    v = mn(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x111, 0xF, 0xF, false));
    v = mn(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x112, 0xF, 0xF, false));
    v = mn(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x114, 0xF, 0xF, false));
    v = mn(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x118, 0xF, 0xF, false));
    uint32_t m = (uint32_t)__builtin_amdgcn_readlane((int)v, 15);
    m = mn(m, (uint32_t)__builtin_amdgcn_readlane((int)v, 31));
    m = mn(m, (uint32_t)__builtin_amdgcn_readlane((int)v, 47));
    return mn(m, (uint32_t)__builtin_amdgcn_readlane((int)v, 63));
}

// Minimum of v over all 64 lanes (every lane active), returned wave-uniform:
// row_shr steps leave each row's minimum in its lane 15, and the four row
// results are read out as scalars.
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
    v = umin64(v, row_down64<1>(v));
    v = umin64(v, row_down64<2>(v));
    v = umin64(v, row_down64<4>(v));
    v = umin64(v, row_down64<8>(v));
    const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    uint64_t m = ~0ull;
#pragma unroll
    for (int r = 15; r < 64; r += 16) {
        const uint64_t x = ((uint64_t)__builtin_amdgcn_readlane(hi, r) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane(lo, r);
        m = umin64(m, x);
    }
    return m;
}

}  // namespace swann
