// The int8 path's activation preparation of one group of 128 or 256
// positions by one wave, shared by the prepare kernel and the engine kernels
// that prepare the next projection's input themselves.
#pragma once

#include "common.h"
#include "wave.h"

namespace nd {

// position p within a row -> byte index in the permuted int8 activation row
__device__ __forceinline__ int permuted_index(int kind, int p) {
    if (kind == kNib) {
        int d = p >> 3, i = p & 7;  // codes 0,2,4,6 then 1,3,5,7 of each 8-code dword
        return (d << 3) | ((i & 1) << 2) | (i >> 1);
    }
    int d = p >> 4, i = p & 15;  // selector m = i&3 holds crumbs m, m+4, m+8, m+12
    return (d << 4) | ((i & 3) << 2) | (i >> 2);
}

// Groups of 8 .. 64 positions: lane t holds position p (groups are aligned
// runs of GROUP lanes): the group FWHT as in-wave butterflies (the
// reference's stage order and operands), the group absmax as an in-wave max,
// then the reference's quantiser (sdot.cpp:56-81: scale = absmax / 127, 1 for
// an all-zero group, absmax if the quotient underflows; q = clamp(rint(x /
// scale), +-127) with IEEE division). The group's first lane stores the scale
// at *xs (and *xst when not null); q goes to qv (the vector's row of dev
// bytes) in the permuted order. Past `padded` a position stores zero. With
// `store` false the lane takes part in the group's arithmetic and stores
// nothing.
template <int GROUP>
__device__ __forceinline__ void prepare_lane(float r, int t, int p, int padded, int dev, float scale, int kind,
                                             int8_t *qv, float *xs, float *xst, bool store = true) {
    wave_butterflies<GROUP, 1>(r, t);
    r = r * scale;
    const float absmax = group_max<GROUP>(fabsf(r), t);
    int8_t out = 0;
    if (p < padded) {
        float sc = absmax > 0 ? absmax / 127 : 1;  // sdot.cpp:77-81
        if (sc == 0.0f) sc = absmax;                // subnormal absmax/127 underflows
        if (store && p % GROUP == 0) {
            *xs = sc;
            if (xst) *xst = sc;
        }
        float val = rintf(r / sc);
        val = val < -127.0f ? -127.0f : (127.0f < val ? 127.0f : val);
        out = static_cast<int8_t>(val);
    }
    if (store && p < dev) qv[permuted_index(kind, p)] = out;
}

// Lane t holds positions base + t + 64 k (k < GROUP / 64) of its wave's group
// in r: the FWHT stages 1 .. 32 run as in-wave butterflies on every k, then
// the stages 64 and 128 between a lane's own values, in the reference's
// stage order and with its operands (x + y, x - y); then the absmax over the
// wave and the reference's quantiser (sdot.cpp:56-81: scale = absmax / 127,
// 1 for an all-zero group, absmax if the quotient underflows; q =
// clamp(rint(x / scale), +-127) with IEEE division). Lane 0 stores the scale
// at *xs (and *xst when not null); the codes go to qv (the vector's row of
// dev bytes) in the permuted order. A group at or past `padded` stores zeros
// and no scale.
template <int GROUP>
__device__ __forceinline__ void prepare_group_wave(float (&r)[GROUP / 64], int t, int base, int padded, int dev,
                                                   float scale, int kind, int8_t *qv, float *xs, float *xst) {
    constexpr int VPL = GROUP / 64;  // values per lane
#pragma unroll
    for (int k = 0; k < VPL; ++k) wave_butterflies<64, 1>(r[k], t);
#pragma unroll
    for (int h = 1; h < VPL; h *= 2)  // stages 64 h
#pragma unroll
        for (int k = 0; k < VPL; ++k)
            if (!(k & h)) {
                const float a = r[k], b = r[k + h];
                r[k] = a + b;
                r[k + h] = a - b;
            }
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        r[k] = r[k] * scale;
        m = fmaxf(m, fabsf(r[k]));
    }
    const float absmax = wave_max(m, t);
    const bool live = base < padded;  // a whole group of the padded length
    float sc = absmax > 0 ? absmax / 127 : 1;  // sdot.cpp:77-81
    if (sc == 0.0f) sc = absmax;                // subnormal absmax/127 underflows
    if (live && t == 0) {
        *xs = sc;
        if (xst) *xst = sc;
    }
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int p = base + t + 64 * k;
        int8_t out = 0;
        if (live) {
            float val = rintf(r[k] / sc);
            val = val < -127.0f ? -127.0f : (127.0f < val ? 127.0f : val);
            out = static_cast<int8_t>(val);
        }
        if (p < dev) qv[permuted_index(kind, p)] = out;
    }
}

}  // namespace nd
