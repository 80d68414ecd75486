// Wave-level exchange helpers for gfx950 (64-lane wavefronts).
#pragma once

#include <hip/hip_runtime.h>

namespace nd {

// Value of the butterfly partner lane t ^ H (H < 64) without LDS round trips:
// DPP quad permutes (1, 2), row shifts (4, 8) and the gfx950 row swaps (16, 32).
template <int H>
__device__ __forceinline__ float butterfly_partner(float v, int t) {
    const int iv = __builtin_bit_cast(int, v);
    if constexpr (H == 1) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
    } else if constexpr (H == 2) {
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
    } else if constexpr (H == 4 || H == 8) {
        const float up = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0x100 + H, 0xF, 0xF, false));
        const float down = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0x110 + H, 0xF, 0xF, false));
        return (t & H) ? down : up;  // row_shl:H reads lane t+H, row_shr:H reads lane t-H
    } else if constexpr (H == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
        return __builtin_bit_cast(float, (t & 16) ? r[0] : r[1]);
    } else {
        static_assert(H == 32, "butterfly stride");
        const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
        return __builtin_bit_cast(float, (t & 32) ? r[0] : r[1]);
    }
}

// In-wave FWHT stages of stride H, 2H, ... < min(GROUP, 64) on lane t's
// value: the reference's butterfly (a + b, a - b) with the same operands
// (cq.cpp:30-46); the lower lane adds its partner, the upper lane adds the
// exactly negated own value, so both results are bit-identical.
template <int GROUP, int H>
__device__ __forceinline__ void wave_butterflies(float &v, int t) {
    if constexpr (H < GROUP && H < 64) {
        const float o = butterfly_partner<H>(v, t);
        const float sv = (t & H) ? -v : v;
        v = o + sv;
        wave_butterflies<GROUP, H * 2>(v, t);
    }
}

// Max over aligned groups of G lanes (G <= 64), result in every lane of the group.
template <int G, int H = 1>
__device__ __forceinline__ float group_max(float v, int t) {
    if constexpr (H < G) {
        v = fmaxf(v, butterfly_partner<H>(v, t));
        return group_max<G, H * 2>(v, t);
    } else {
        return v;
    }
}

// Max / sum over the 64 lanes, result in every lane (xor butterflies).
__device__ __forceinline__ float wave_max(float v, int t) {
    v = fmaxf(v, butterfly_partner<1>(v, t));
    v = fmaxf(v, butterfly_partner<2>(v, t));
    v = fmaxf(v, butterfly_partner<4>(v, t));
    v = fmaxf(v, butterfly_partner<8>(v, t));
    v = fmaxf(v, butterfly_partner<16>(v, t));
    return fmaxf(v, butterfly_partner<32>(v, t));
}
__device__ __forceinline__ float wave_sum(float v, int t) {
    v += butterfly_partner<1>(v, t);
    v += butterfly_partner<2>(v, t);
    v += butterfly_partner<4>(v, t);
    v += butterfly_partner<8>(v, t);
    v += butterfly_partner<16>(v, t);
    return v + butterfly_partner<32>(v, t);
}

// Index of the job whose workgroup range holds `blk` in a job table sorted by
// block_begin (jobs[0] begins at 0): the last j with jobs[j].block_begin <=
// blk, by binary search, so a table of one job per (token, matrix piece)
// costs a few scalar loads per workgroup rather than one per job.
template <class P>
__device__ __forceinline__ int find_job(P jobs, int njobs, int blk) {
    int lo = 0, hi = njobs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (jobs[mid].block_begin <= blk) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

}  // namespace nd
