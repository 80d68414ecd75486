// gfx950 kernels for the int8 ("SDOT-equivalent") CQ path.
//
// Activations: after the per-group FWHT (shared with the FP32 path), each
// group is quantized exactly as sdot.cpp:77-81 does: absmax, scale =
// absmax/127 (1 if absmax == 0; absmax if the quotient underflows),
// q = clamp(rint(x/scale), +-127) with IEEE division. q is stored in a lane
// order matched to the code decode below, so every int8 product pairs the
// right code with the right activation.
//
// GEMV: one lane per output row, codes chunk-major (common.h). Codes become
// int8 centroids with v_perm_b32 byte lookups (three perms per four 4-bit
// codes, one per four 2-bit codes) and are multiplied with v_dot4_i32_i8
// against activations staged in LDS per workgroup (wave-uniform reads).
// The int32 group dot is exact in any order; the epilogue is the reference's
//   value += (float(dot) * (half(norm) * cs)) * x_scale[g]
// sequentially over g (sdot.cpp:43-44, 142-149), so outputs are bit-exact.
#include "common.h"
#include "sdot_prepare.h"
#include "wave.h"

#include <hip/hip_fp16.h>

#include <cstdlib>
#include <cstring>
#include <type_traits>

namespace nd {

namespace {

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// One block per (segment of positions, vector). seg = max(256, group).
__global__ __launch_bounds__(256) void sdot_quantize_kernel(const float *__restrict__ rot, int rot_stride, int padded,
                                                            int dev, int group, int kind, int8_t *__restrict__ q,
                                                            float *__restrict__ xs, int groups, int seg) {
    __shared__ unsigned gmax[32];
    const int v = blockIdx.y;
    const int base = blockIdx.x * seg;
    const int ngroups = seg / group > 0 ? seg / group : 1;  // groups in this segment (<= 32)
    for (int i = threadIdx.x; i < ngroups; i += blockDim.x) gmax[i] = 0u;
    __syncthreads();
    const float *rv = rot + static_cast<size_t>(v) * rot_stride;
    for (int i = threadIdx.x; i < seg; i += blockDim.x) {
        int p = base + i;
        if (p < padded) atomicMax(&gmax[i / group], __float_as_uint(fabsf(rv[p])));
    }
    __syncthreads();
    int8_t *qv = q + static_cast<size_t>(v) * dev;
    for (int i = threadIdx.x; i < seg; i += blockDim.x) {
        int p = base + i;
        if (p >= dev) continue;
        int8_t out = 0;
        if (p < padded) {
            float absmax = __uint_as_float(gmax[i / group]);
            float scale = absmax > 0 ? absmax / 127 : 1;
            if (scale == 0.0f) scale = absmax;  // subnormal absmax/127 underflows
            if (p % group == 0) xs[static_cast<size_t>(v) * groups + p / group] = scale;
            float val = rintf(rv[p] / scale);
            val = val < -127.0f ? -127.0f : (127.0f < val ? 127.0f : val);
            out = static_cast<int8_t>(val);
        }
        qv[permuted_index(kind, p)] = out;
    }
}

// Fused prepare: one block per (segment of positions, vector). The FWHT
// runs in LDS with the reference's stage order (cq.cpp:30-46: h = 1, 2, ...,
// (a + b, a - b), then one multiply by 1/sqrt(group)), so the rotated values,
// and from them the int8 codes and scales, are bit-identical to a separate
// transform followed by sdot_quantize_kernel. seg = max(group, 1024).
constexpr int kPrepareMaxGroup = kSdotFusedPrepareMaxGroup;
constexpr int kPrepareMinSeg = 1024;

__global__ __launch_bounds__(256) void sdot_prepare_kernel(const float *__restrict__ x0,
                                                           const float *const *__restrict__ xptr, int batch, int in,
                                                           int padded, int dev, int group, float scale, int kind,
                                                           int8_t *__restrict__ q, float *__restrict__ xs,
                                                           float *__restrict__ xst, int groups, int seg) {
    extern __shared__ float buf[];
    __shared__ unsigned gmax[kPrepareMinSeg / 8];
    const int v = blockIdx.y;
    const int base = blockIdx.x * seg;
    const int ngroups = seg / group;  // whole groups: seg is a multiple of group
    const float *xv = (xptr ? xptr[v / batch] : x0) + static_cast<size_t>(v % batch) * in;
    for (int i = threadIdx.x; i < ngroups; i += blockDim.x) gmax[i] = 0u;
    for (int i = threadIdx.x; i < seg; i += blockDim.x) {
        const int p = base + i;
        buf[i] = p < in ? xv[p] : 0.0f;
    }
    __syncthreads();
    for (int h = 1; h < group; h <<= 1) {
        for (int t = threadIdx.x; t < seg / 2; t += blockDim.x) {
            const int lo = (t / h) * 2 * h + (t % h);
            const float a = buf[lo], b = buf[lo + h];
            buf[lo] = a + b;
            buf[lo + h] = a - b;
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < seg; i += blockDim.x) {
        const float r = buf[i] * scale;
        buf[i] = r;
        if (base + i < padded) atomicMax(&gmax[i / group], __float_as_uint(fabsf(r)));
    }
    __syncthreads();
    int8_t *qv = q + static_cast<size_t>(v) * dev;
    for (int i = threadIdx.x; i < seg; i += blockDim.x) {
        const int p = base + i;
        if (p >= dev) break;
        int8_t out = 0;
        if (p < padded) {
            const float absmax = __uint_as_float(gmax[i / group]);
            float sc = absmax > 0 ? absmax / 127 : 1;  // sdot.cpp:77-81
            if (sc == 0.0f) sc = absmax;                // subnormal absmax/127 underflows
            if (p % group == 0) {
                xs[static_cast<size_t>(v) * groups + p / group] = sc;
                if (xst) xst[(static_cast<size_t>(v / batch) * groups + p / group) * batch + v % batch] = sc;
            }
            float val = rintf(buf[i] / sc);
            val = val < -127.0f ? -127.0f : (127.0f < val ? 127.0f : val);
            out = static_cast<int8_t>(val);
        }
        qv[permuted_index(kind, p)] = out;
    }
}

// ---------------------------------------------------------------------------
// GEMV
// ---------------------------------------------------------------------------
// 8 four-bit codes (one dword) -> int8 centroids for codes {0,2,4,6} and {1,3,5,7}.
// (x & m) | c in one VALU op (the compiler emits a separate and + or); GFX9
// VALU takes one scalar operand, so the mask comes in a VGPR.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m_vgpr, uint32_t c_sgpr) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m_vgpr), "s"(c_sgpr));
    return r;
}

// 13 VALU ops: 3 masks/shifts for the low-bit selectors, 4 for the high-half
// selectors, 6 byte permutes.
__device__ __forceinline__ void decode_nib(uint32_t w, uint32_t T0, uint32_t T1, uint32_t T2, uint32_t T3,
                                           uint32_t &ce, uint32_t &co) {
    const uint32_t m4 = 0x04040404u;
    const uint32_t w4 = w >> 4;
    const uint32_t e = w & 0x07070707u, o = w4 & 0x07070707u;
    const uint32_t le = __builtin_amdgcn_perm(T1, T0, e), he = __builtin_amdgcn_perm(T3, T2, e);
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, o), ho = __builtin_amdgcn_perm(T3, T2, o);
    const uint32_t se = and_or(w >> 1, m4, 0x03020100u);  // bit 3 of each code picks the high half
    const uint32_t so = and_or(w4 >> 1, m4, 0x03020100u);
    ce = __builtin_amdgcn_perm(he, le, se);
    co = __builtin_amdgcn_perm(ho, lo, so);
}

template <int KIND, int GROUP>
struct SdotWindow {
    static constexpr int kChunks = kWindow / (KIND == kNib ? 32 : 64);
    static constexpr int kNorms = GROUP > 0 ? kWindow / GROUP : 1;
    u32x4 codes[kChunks];
    uint16_t norms[kNorms];
};

// Buffer loads with a wave-uniform soffset and one shared per-lane voffset;
// group indices are clamped (phantom groups past the last are never closed).
template <int KIND, int GROUP>
__device__ __forceinline__ void sdot_load(SdotWindow<KIND, GROUP> &st, __amdgpu_buffer_rsrc_t codes,
                                          __amdgpu_buffer_rsrc_t norms, int w, int groups, int wpg) {
    constexpr int C = SdotWindow<KIND, GROUP>::kChunks;
    constexpr int NN = SdotWindow<KIND, GROUP>::kNorms;
    constexpr int CS = kRowsPerBlock * 16, NS = kRowsPerBlock * 2;  // tile strides of a chunk / a group
    const uint32_t code_lane = threadIdx.x * 16u, norm_lane = threadIdx.x * 2u;
#pragma unroll
    for (int c = 0; c < C; ++c)
        st.codes[c] = __builtin_amdgcn_raw_buffer_load_b128(codes, code_lane, (w * C + c) * CS, kStreamLoad);
    if constexpr (GROUP > 0) {
#pragma unroll
        for (int k = 0; k < NN; ++k)
            st.norms[k] = __builtin_amdgcn_raw_buffer_load_b16(norms, norm_lane, min(w * NN + k, groups - 1) * NS, 0);
    } else {
        st.norms[0] = __builtin_amdgcn_raw_buffer_load_b16(norms, norm_lane, min(w / wpg, groups - 1) * NS, 0);
    }
}

// Per window and batch row, the permuted int8 activations (kWindow/4 dwords)
// and the group scales closing in the window are staged in LDS once per
// workgroup and read back as wave-uniform (broadcast) loads.
template <int GROUP, int BT>
struct Stage {
    static constexpr int kQ = kWindow / 4;                               // dwords per batch row
    static constexpr int kXs = GROUP > 0 ? kWindow / GROUP : 1;          // scales per batch row
    static constexpr int kQ4 = BT * kQ / 4;                              // uint4 per window
    static constexpr int kXsAll = BT * kXs;
};

template <int GROUP, int BT>
struct StageRegs {
    static constexpr int kQn = (Stage<GROUP, BT>::kQ4 + kRowsPerBlock - 1) / kRowsPerBlock;
    static constexpr int kXsn = (Stage<GROUP, BT>::kXsAll + kRowsPerBlock - 1) / kRowsPerBlock;
    u32x4 q[kQn];
    float xs[kXsn];
};

// Thread t fetches staged items t, t + blockDim, ... of window w.
template <int GROUP, int BT>
__device__ __forceinline__ void stage_load(StageRegs<GROUP, BT> &r, __amdgpu_buffer_rsrc_t q,
                                           __amdgpu_buffer_rsrc_t xs, int qdw, int groups, int w, int wpg) {
    using S = Stage<GROUP, BT>;
    const int t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < StageRegs<GROUP, BT>::kQn; ++k) {
        const int i = t + k * kRowsPerBlock;  // uint4 index within the window
        const int b = i / (S::kQ / 4), j = i % (S::kQ / 4);
        // Indices past the window get an offset beyond the buffer bound: the
        // load returns zero without a memory request. Every thread loads and
        // stores, so the loads stay where they are issued.
        const uint32_t off = i < S::kQ4 ? (b * qdw + w * S::kQ + j * 4) * 4u : 0x80000000u;
        r.q[k] = __builtin_amdgcn_raw_buffer_load_b128(q, off, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < StageRegs<GROUP, BT>::kXsn; ++k) {
        const int i = t + k * kRowsPerBlock;
        const int b = i / S::kXs, gi = i % S::kXs;
        const int g = GROUP > 0 ? min(w * S::kXs + gi, groups - 1) : min(w / wpg, groups - 1);
        const uint32_t off = i < S::kXsAll ? (b * groups + g) * 4u : 0x80000000u;
        r.xs[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xs, off, 0, 0));
    }
}

template <int GROUP, int BT>
__device__ __forceinline__ void stage_store(const StageRegs<GROUP, BT> &r, u32x4 *lq, float *lxs) {
    using S = Stage<GROUP, BT>;
    const int t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < StageRegs<GROUP, BT>::kQn; ++k) lq[t + k * kRowsPerBlock] = r.q[k];
#pragma unroll
    for (int k = 0; k < StageRegs<GROUP, BT>::kXsn; ++k) lxs[t + k * kRowsPerBlock] = r.xs[k];
}

// One window: decode each code dword once, dot it against BT batch rows.
template <int KIND, int GROUP, int BT>
__device__ __forceinline__ void sdot_compute(const SdotWindow<KIND, GROUP> &st, const u32x4 *lq, const float *lxs,
                                             const uint32_t cent[4], float cs, float (&value)[BT], int (&dot)[BT],
                                             int w, int groups, int wpg) {
    using S = Stage<GROUP, BT>;
    constexpr int C = SdotWindow<KIND, GROUP>::kChunks;
    constexpr int NN = SdotWindow<KIND, GROUP>::kNorms;
    const int gbase = w * NN;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const uint32_t words[4] = {st.codes[c].x, st.codes[c].y, st.codes[c].z, st.codes[c].w};
        // this chunk's activations: 8 (4-bit) or 16 (2-bit) dwords per batch row
        constexpr int QPC = KIND == kNib ? 8 : 16;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t wd = words[d];
            if constexpr (KIND == kNib) {
                uint32_t ce, co;
                decode_nib(wd, cent[0], cent[1], cent[2], cent[3], ce, co);
#pragma unroll
                for (int b = 0; b < BT; ++b) {
                    const uint32_t *qb = reinterpret_cast<const uint32_t *>(lq + b * (S::kQ / 4)) + c * QPC + d * 2;
                    dot[b] = __builtin_amdgcn_sdot4(static_cast<int>(ce), static_cast<int>(qb[0]), dot[b], false);
                    dot[b] = __builtin_amdgcn_sdot4(static_cast<int>(co), static_cast<int>(qb[1]), dot[b], false);
                }
            } else {
                uint32_t cc[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) cc[m] = __builtin_amdgcn_perm(0u, cent[0], (wd >> (2 * m)) & 0x03030303u);
#pragma unroll
                for (int b = 0; b < BT; ++b) {
                    const uint32_t *qb = reinterpret_cast<const uint32_t *>(lq + b * (S::kQ / 4)) + c * QPC + d * 4;
#pragma unroll
                    for (int m = 0; m < 4; ++m)
                        dot[b] = __builtin_amdgcn_sdot4(static_cast<int>(cc[m]), static_cast<int>(qb[m]), dot[b], false);
                }
            }
            if constexpr (GROUP > 0) {
                const int pos_end = (c * 4 + d + 1) * (KIND == kNib ? 8 : 16);
                if (pos_end % GROUP == 0) {
                    const int k = pos_end / GROUP - 1;
                    // A select rather than a branch: the norm is used on every
                    // path, so its load is never sunk next to its use.
                    const bool real = gbase + k < groups;
                    const float ns = h2f(st.norms[k]) * cs;  // sdot.cpp:43-44
#pragma unroll
                    for (int b = 0; b < BT; ++b) {
                        const float sum = value[b] + (static_cast<float>(dot[b]) * ns) * lxs[b * S::kXs + k];
                        value[b] = real ? sum : value[b];
                    }
#pragma unroll
                    for (int b = 0; b < BT; ++b) dot[b] = 0;
                }
            }
        }
    }
    if constexpr (GROUP == 0) {
        if ((w + 1) % wpg == 0) {
            const bool real = w / wpg < groups;
            const float ns = h2f(st.norms[0]) * cs;
#pragma unroll
            for (int b = 0; b < BT; ++b) {
                const float sum = value[b] + (static_cast<float>(dot[b]) * ns) * lxs[b];
                value[b] = real ? sum : value[b];
            }
#pragma unroll
            for (int b = 0; b < BT; ++b) dot[b] = 0;
        }
    }
}

// Batch rows [b_begin, b_end) in tiles of BT; one lane per output row.
template <int KIND, int GROUP, int BT>
__global__ __launch_bounds__(kRowsPerBlock, 2) void sdot_gemv_kernel(SdotJob job0, const SdotJob *__restrict__ jobs,
                                                                     int njobs, SdotGeom geom, int b_begin, int b_end) {
    using S = Stage<GROUP, BT>;
    // staging buffers padded to whole blocks: every thread stores its slots
    __shared__ u32x4 lq[2][StageRegs<GROUP, BT>::kQn * kRowsPerBlock];
    __shared__ float lxs[2][StageRegs<GROUP, BT>::kXsn * kRowsPerBlock];
    const int blk = blockIdx.x;
    SdotJob J = job0;
    if (njobs > 0) {
        const ND_CONST SdotJob *cj = (const ND_CONST SdotJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J.codes = cj[j].codes;
        J.norms = cj[j].norms;
        J.q = cj[j].q;
        J.xs = cj[j].xs;
        J.y = cj[j].y;
        J.rows = cj[j].rows;
        J.n_pad = cj[j].n_pad;
        J.block_begin = cj[j].block_begin;
        J.batch = cj[j].batch;
        J.ystride = cj[j].ystride;
    }
    const int rows = J.rows;
    const size_t ystride = J.ystride ? J.ystride : rows;
    const int tile = blk - J.block_begin;
    const int row = tile * kRowsPerBlock + threadIdx.x;
    const int windows = geom.windows, groups = geom.groups;
    const int wpg = GROUP == 0 ? geom.group / kWindow : 1;
    const int qdw = windows * (kWindow / 4);  // int32 activation words per batch row
    const uint32_t cent[4] = {geom.cent[0], geom.cent[1], geom.cent[2], geom.cent[3]};
    const float cs = geom.centroid_scale;
    // this workgroup's row tile of codes and norms
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms = buffer_rsrc(J.norms + static_cast<size_t>(tile) * groups * kRowsPerBlock,
                                                     static_cast<uint32_t>(groups) * kRowsPerBlock * 2u);

    // one batch tile per blockIdx.y (b_end bounds the tiles this launch covers)
    for (int b0 = b_begin + static_cast<int>(blockIdx.y) * BT; b0 < b_end; b0 += BT * static_cast<int>(gridDim.y)) {
        const __amdgpu_buffer_rsrc_t q = buffer_rsrc(J.q + static_cast<size_t>(b0) * qdw, static_cast<uint32_t>(BT) * qdw * 4u);
        const __amdgpu_buffer_rsrc_t xs = buffer_rsrc(J.xs + static_cast<size_t>(b0) * groups, static_cast<uint32_t>(BT) * groups * 4u);
        SdotWindow<KIND, GROUP> cur, nxt;
        StageRegs<GROUP, BT> sr;
        stage_load<GROUP, BT>(sr, q, xs, qdw, groups, 0, wpg);
        sdot_load<KIND, GROUP>(cur, codes, norms, 0, groups, wpg);
        __syncthreads();  // previous tile finished reading stage buffer 0
        stage_store<GROUP, BT>(sr, lq[0], lxs[0]);
        __syncthreads();
        float value[BT];
        int dot[BT];
#pragma unroll
        for (int b = 0; b < BT; ++b) {
            value[b] = 0.0f;
            dot[b] = 0;
        }
        // Per window: issue the next window's staged activations and codes
        // (unconditional, clamped), compute this window, store the next
        // staging buffer, one barrier. Pairs of windows run in a loop with a
        // single exit (no mid-body break), so the loop header is reached only
        // from the loop itself and the prologue; an odd last window follows.
        int w = 0;
        for (; w + 1 < windows; w += 2) {
            stage_load<GROUP, BT>(sr, q, xs, qdw, groups, w + 1, wpg);
            sdot_load<KIND, GROUP>(nxt, codes, norms, w + 1, groups, wpg);
            asm volatile("" ::: "memory");  // keep the next window's loads ahead of this compute
            sdot_compute<KIND, GROUP, BT>(cur, lq[0], lxs[0], cent, cs, value, dot, w, groups, wpg);
            stage_store<GROUP, BT>(sr, lq[1], lxs[1]);
            __syncthreads();
            const int w2 = min(w + 2, windows - 1);
            stage_load<GROUP, BT>(sr, q, xs, qdw, groups, w2, wpg);
            sdot_load<KIND, GROUP>(cur, codes, norms, w2, groups, wpg);
            asm volatile("" ::: "memory");
            sdot_compute<KIND, GROUP, BT>(nxt, lq[1], lxs[1], cent, cs, value, dot, w + 1, groups, wpg);
            stage_store<GROUP, BT>(sr, lq[0], lxs[0]);  // window w2 (re-staged if it is the last)
            __syncthreads();
        }
        if (w < windows) sdot_compute<KIND, GROUP, BT>(cur, lq[0], lxs[0], cent, cs, value, dot, w, groups, wpg);
        if (row < rows) {
#pragma unroll
            for (int b = 0; b < BT; ++b) ((ND_GLOBAL float *)J.y)[static_cast<size_t>(b0 + b) * ystride + row] = value[b];
        }
    }
}

template <int KIND, int BT>
void launch_sdot_bt(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int b0,
                    int b1, hipStream_t s) {
    dim3 grid(blocks, (b1 - b0) / BT), block(kRowsPerBlock);
    switch (g.group > kWindow ? 0 : g.group) {
    case 8:
        if constexpr (KIND == kNib) {
            hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 8, BT>), grid, block, 0, s, job0, jobs, njobs, g, b0, b1);
            break;
        }
        [[fallthrough]];
    case 16: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 16, BT>), grid, block, 0, s, job0, jobs, njobs, g, b0, b1); break;
    case 32: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 32, BT>), grid, block, 0, s, job0, jobs, njobs, g, b0, b1); break;
    case 64: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 64, BT>), grid, block, 0, s, job0, jobs, njobs, g, b0, b1); break;
    case 128: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 128, BT>), grid, block, 0, s, job0, jobs, njobs, g, b0, b1); break;
    case 256: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 256, BT>), grid, block, 0, s, job0, jobs, njobs, g, b0, b1); break;
    default: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 0, BT>), grid, block, 0, s, job0, jobs, njobs, g, b0, b1); break;
    }
    ND_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// int8 path on MFMA (batch >= 2, groups of 32 .. 256 positions)
//
// One wave per (32 weight rows, 32 batch rows) and v_mfma_i32_32x32x32_i8
// per 32 positions: B = decoded int8 centroids of weight row lane % 32,
// A = the permuted int8 activations of batch row lane % 32; lanes 0-31 and
// 32-63 cover positions 0-15 and 16-31 of the step, in the same byte order
// for A and B (the sum over K is independent of how K is laid out across a
// lane's bytes, as long as A and B agree). The accumulator of a group is the
// exact int32 group dot, so the epilogue is the reference's
//   value += (float(dot) * (half(norm) * cs)) * x_scale[g]
// in group order (sdot.cpp:43-44, 142-149): bit-identical outputs.
// Accumulator register r of lane l holds batch row 8(r/4) + 4(l/32) + r%4
// and weight row l % 32; J = 1, 2, 4 keeps the 4, 8 or 16 registers that
// cover the batch tile. Codes, activations, norms and the transposed scales
// of three groups are in flight per lane (a register ring); loads past the
// row tile, the batch tile or the last group read zero through the buffer
// bounds or land on data that is never used.
// ---------------------------------------------------------------------------
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int KIND, int GROUP, int J>
struct MfmaSlot {
    static constexpr int kSteps = GROUP / 32;
    static constexpr int kCodeDw = KIND == kNib ? 2 : 1;  // code dwords per lane per step
    uint32_t code[kSteps * kCodeDw];
    u32x4 q[kSteps];
    u32x4 xs[J];
    uint16_t norm;
};

template <int KIND, int GROUP, int J>
__device__ __forceinline__ void mfma_load(MfmaSlot<KIND, GROUP, J> &sl, __amdgpu_buffer_rsrc_t codes,
                                          __amdgpu_buffer_rsrc_t norms, __amdgpu_buffer_rsrc_t q,
                                          __amdgpu_buffer_rsrc_t xst, int g, int rt, int i, int h, int dev,
                                          int batch, int b0) {
    using S = MfmaSlot<KIND, GROUP, J>;
#pragma unroll
    for (int st = 0; st < S::kSteps; ++st) {
        const int pos = g * GROUP + st * 32;  // first position of the step
        if constexpr (KIND == kNib) {
            // chunk = 32 positions; this lane's dwords 2h, 2h+1
            const int soff = __builtin_amdgcn_readfirstlane((pos / 32) * kRowsPerBlock * 16);
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(codes, rt * 16u + h * 8u, soff, 0);
            sl.code[2 * st] = v[0];
            sl.code[2 * st + 1] = v[1];
        } else {
            // chunk = 64 positions; this step is dwords 2((pos / 32) % 2) .. +1; this lane's is + h
            const int soff = __builtin_amdgcn_readfirstlane((pos / 64) * kRowsPerBlock * 16 + ((pos / 32) % 2) * 8);
            sl.code[st] = __builtin_amdgcn_raw_buffer_load_b32(codes, rt * 16u + h * 4u, soff, 0);
        }
        sl.q[st] = __builtin_amdgcn_raw_buffer_load_b128(q, static_cast<uint32_t>(i) * dev + h * 16u,
                                                         __builtin_amdgcn_readfirstlane(pos), 0);
    }
#pragma unroll
    for (int j = 0; j < J; ++j)
        sl.xs[j] = __builtin_amdgcn_raw_buffer_load_b128(
            xst, (b0 + 8 * j + 4 * h) * 4u, __builtin_amdgcn_readfirstlane(g * batch * 4), 0);
    sl.norm = __builtin_amdgcn_raw_buffer_load_b16(norms, rt * 2u,
                                                   __builtin_amdgcn_readfirstlane(g * kRowsPerBlock * 2), 0);
}

// mfma_load for one batch row prepared in LDS (qst: the row's permuted codes,
// dev bytes; scst: its group scales): lane (i, h) takes what mfma_load's
// buffer loads would return for batch row i < 1, zeros for the rows past it.
template <int KIND, int GROUP, int J>
__device__ __forceinline__ void mfma_load_x(MfmaSlot<KIND, GROUP, J> &sl, __amdgpu_buffer_rsrc_t codes,
                                            __amdgpu_buffer_rsrc_t norms, const int8_t *qst, const float *scst,
                                            int g, int rt, int i, int h, int dev, int groups) {
    using S = MfmaSlot<KIND, GROUP, J>;
#pragma unroll
    for (int st = 0; st < S::kSteps; ++st) {
        const int pos = g * GROUP + st * 32;
        if constexpr (KIND == kNib) {
            const int soff = __builtin_amdgcn_readfirstlane((pos / 32) * kRowsPerBlock * 16);
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(codes, rt * 16u + h * 8u, soff, 0);
            sl.code[2 * st] = v[0];
            sl.code[2 * st + 1] = v[1];
        } else {
            const int soff = __builtin_amdgcn_readfirstlane((pos / 64) * kRowsPerBlock * 16 + ((pos / 32) % 2) * 8);
            sl.code[st] = __builtin_amdgcn_raw_buffer_load_b32(codes, rt * 16u + h * 4u, soff, 0);
        }
        sl.q[st] = i == 0 && pos < dev ? *reinterpret_cast<const u32x4 *>(qst + pos + h * 16) : u32x4{0u, 0u, 0u, 0u};
    }
    const uint32_t sc = g < groups ? __builtin_bit_cast(uint32_t, scst[g < groups ? g : 0]) : 0u;
#pragma unroll
    for (int j = 0; j < J; ++j) sl.xs[j] = u32x4{j == 0 && h == 0 ? sc : 0u, 0u, 0u, 0u};
    sl.norm = __builtin_amdgcn_raw_buffer_load_b16(norms, rt * 2u,
                                                   __builtin_amdgcn_readfirstlane(g * kRowsPerBlock * 2), 0);
}

template <int KIND, int GROUP, int J>
__device__ __forceinline__ void mfma_group(const MfmaSlot<KIND, GROUP, J> &sl, const uint32_t cent[4], float cs,
                                           float (&value)[4 * J]) {
    using S = MfmaSlot<KIND, GROUP, J>;
    v16i acc = {};
#pragma unroll
    for (int st = 0; st < S::kSteps; ++st) {
        v4i b;
        if constexpr (KIND == kNib) {
            uint32_t ce0, co0, ce1, co1;
            decode_nib(sl.code[2 * st], cent[0], cent[1], cent[2], cent[3], ce0, co0);
            decode_nib(sl.code[2 * st + 1], cent[0], cent[1], cent[2], cent[3], ce1, co1);
            b = v4i{static_cast<int>(ce0), static_cast<int>(co0), static_cast<int>(ce1), static_cast<int>(co1)};
        } else {
            const uint32_t wd = sl.code[st];
#pragma unroll
            for (int m = 0; m < 4; ++m) b[m] = static_cast<int>(__builtin_amdgcn_perm(0u, cent[0], (wd >> (2 * m)) & 0x03030303u));
        }
        const v4i a = __builtin_bit_cast(v4i, sl.q[st]);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc, 0, 0, 0);
    }
    const float ns = h2f(sl.norm) * cs;  // sdot.cpp:43-44
#pragma unroll
    for (int j = 0; j < J; ++j) {
        // bit_cast the whole vector: this compiler's __builtin_bit_cast of a
        // single ext_vector element lvalue (v.y, v[t]) reads element 0
        const f32x4 xs = __builtin_bit_cast(f32x4, sl.xs[j]);
#pragma unroll
        for (int t = 0; t < 4; ++t) value[4 * j + t] = value[4 * j + t] + (static_cast<float>(acc[4 * j + t]) * ns) * xs[t];
    }
}

constexpr int kMfmaRing = 3;

template <int KIND, int GROUP, int J>
__global__ __launch_bounds__(kRowsPerBlock) void sdot_mfma_kernel(SdotJob job0, const SdotJob *__restrict__ jobs,
                                                                  int njobs, SdotGeom geom) {
    const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);      // wave-uniform
    const int rb = blockIdx.x * (kRowsPerBlock / 64) + wave;                // 32-row block across the plan
    const int blk = rb / (kRowsPerBlock / 32);                            // 256-row tile across the plan
    SdotJob J0 = job0;
    if (njobs > 0) {
        const ND_CONST SdotJob *cj = (const ND_CONST SdotJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J0.codes = cj[j].codes;
        J0.norms = cj[j].norms;
        J0.q = cj[j].q;
        J0.y = cj[j].y;
        J0.rows = cj[j].rows;
        J0.block_begin = cj[j].block_begin;
        J0.batch = cj[j].batch;
        J0.ystride = cj[j].ystride;
        J0.xst = cj[j].xst;
    }
    const int rows = J0.rows, batch = J0.batch;
    const int tile = blk - J0.block_begin;
    const int rt = (rb % (kRowsPerBlock / 32)) * 32 + i;  // row within the tile
    const int row = tile * kRowsPerBlock + rt;
    const int b0 = static_cast<int>(blockIdx.y) * 32;
    const int groups = geom.groups;
    const int dev = geom.windows * kWindow;
    const uint32_t cent[4] = {geom.cent[0], geom.cent[1], geom.cent[2], geom.cent[3]};
    const float cs = geom.centroid_scale;
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J0.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms = buffer_rsrc(J0.norms + static_cast<size_t>(tile) * groups * kRowsPerBlock,
                                                     static_cast<uint32_t>(groups) * kRowsPerBlock * 2u);
    const int tile_rows = min(32, batch - b0);
    const __amdgpu_buffer_rsrc_t q =
        buffer_rsrc(reinterpret_cast<const int8_t *>(J0.q) + static_cast<size_t>(b0) * dev,
                    static_cast<uint32_t>(tile_rows) * dev);
    const __amdgpu_buffer_rsrc_t xst = buffer_rsrc(J0.xst, static_cast<uint32_t>(groups) * batch * 4u);

    float value[4 * J];
#pragma unroll
    for (int r = 0; r < 4 * J; ++r) value[r] = 0.0f;
    MfmaSlot<KIND, GROUP, J> ring[kMfmaRing];
#pragma unroll
    for (int k = 0; k < kMfmaRing; ++k) mfma_load(ring[k], codes, norms, q, xst, k, rt, i, h, dev, batch, b0);
    // whole rounds of kMfmaRing groups, each slot refilled kMfmaRing groups ahead once used
    int g = 0;
    for (; g + kMfmaRing <= groups; g += kMfmaRing) {
#pragma unroll
        for (int k = 0; k < kMfmaRing; ++k) {
            mfma_group(ring[k], cent, cs, value);
            mfma_load(ring[k], codes, norms, q, xst, g + k + kMfmaRing, rt, i, h, dev, batch, b0);
        }
    }
#pragma unroll
    for (int k = 0; k < kMfmaRing; ++k)
        if (g + k < groups) mfma_group(ring[k], cent, cs, value);
    if (row < rows) {
#pragma unroll
        for (int r = 0; r < 4 * J; ++r) {
            const int m = b0 + 8 * (r / 4) + 4 * h + (r % 4);
            if (m < batch) ((ND_GLOBAL float *)J0.y)[static_cast<size_t>(m) * (J0.ystride ? J0.ystride : rows) + row] = value[r];
        }
    }
}

template <int KIND, int J>
void launch_sdot_mfma_j(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int batch,
                        hipStream_t s) {
    dim3 grid(blocks * (kRowsPerBlock / 128), (batch + 31) / 32), block(kRowsPerBlock);
    switch (g.group) {
    case 32: hipLaunchKernelGGL((sdot_mfma_kernel<KIND, 32, J>), grid, block, 0, s, job0, jobs, njobs, g); break;
    case 64: hipLaunchKernelGGL((sdot_mfma_kernel<KIND, 64, J>), grid, block, 0, s, job0, jobs, njobs, g); break;
    case 128: hipLaunchKernelGGL((sdot_mfma_kernel<KIND, 128, J>), grid, block, 0, s, job0, jobs, njobs, g); break;
    default: hipLaunchKernelGGL((sdot_mfma_kernel<KIND, 256, J>), grid, block, 0, s, job0, jobs, njobs, g); break;
    }
    ND_HIP(hipGetLastError());
}

template <int KIND>
void launch_sdot_mfma(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int batch,
                      hipStream_t s) {
    if (batch <= 8) launch_sdot_mfma_j<KIND, 1>(g, job0, jobs, njobs, blocks, batch, s);
    else if (batch <= 16) launch_sdot_mfma_j<KIND, 2>(g, job0, jobs, njobs, blocks, batch, s);
    else launch_sdot_mfma_j<KIND, 4>(g, job0, jobs, njobs, blocks, batch, s);
}

// ---------------------------------------------------------------------------
// int8 GEMV for one batch row (decode), one thread per output row.
//
// The row's permuted int8 activations and group scales (a few KiB) are
// staged in LDS once per workgroup; after that barrier the waves never
// synchronise again. Each thread streams its row's 16-byte code chunks
// through a register ring kRowRing chunks deep (a chunk is refilled right
// after it is decoded, so loads run continuously ahead), decodes every code
// dword once (v_perm_b32 centroid lookups) and accumulates v_dot4_i32_i8
// against wave-uniform LDS reads. Groups close with the reference's epilogue
//   value += (float(dot) * (half(norm) * cs)) * x_scale[g]
// in group order (sdot.cpp:43-44, 142-149): bit-identical outputs.
// ---------------------------------------------------------------------------
constexpr int kRowRing = 8;
constexpr int kRowMaxDev = 32768;  // staged activation bytes per workgroup

template <int KIND, int GROUP>
struct RowSlot {
    static constexpr int kCodes = KIND == kNib ? 32 : 64;                // codes per chunk
    static constexpr int kNorms = GROUP >= kCodes ? 1 : kCodes / GROUP;  // norms a chunk needs
    u32x4 code;
    uint16_t norm[kNorms];
};

template <int KIND, int GROUP>
__device__ __forceinline__ void row_load(RowSlot<KIND, GROUP> &sl, __amdgpu_buffer_rsrc_t codes,
                                         __amdgpu_buffer_rsrc_t norms, int c, int groups) {
    using S = RowSlot<KIND, GROUP>;
    sl.code = __builtin_amdgcn_raw_buffer_load_b128(codes, threadIdx.x * 16u,
                                                   __builtin_amdgcn_readfirstlane(c * kRowsPerBlock * 16), kStreamLoad);
#pragma unroll
    for (int k = 0; k < S::kNorms; ++k) {
        // the chunk's group (GROUP >= chunk) or its k-th group; phantom groups past the last read the last
        const int g = min(c * S::kCodes / GROUP + k, groups - 1);
        sl.norm[k] = __builtin_amdgcn_raw_buffer_load_b16(
            norms, threadIdx.x * 2u, __builtin_amdgcn_readfirstlane(g * kRowsPerBlock * 2), 0);
    }
}

template <int KIND, int GROUP, bool DOTS>
__device__ __forceinline__ void row_compute(const RowSlot<KIND, GROUP> &sl, const uint32_t *lq, const float *lxs,
                                            const uint32_t cent[4], float cs, int c, int groups, float &value,
                                            int &dot, int32_t *dots_row) {
    using S = RowSlot<KIND, GROUP>;
    const uint32_t words[4] = {sl.code.x, sl.code.y, sl.code.z, sl.code.w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        if constexpr (KIND == kNib) {
            uint32_t ce, co;
            decode_nib(words[d], cent[0], cent[1], cent[2], cent[3], ce, co);
            const uint32_t *qd = lq + c * 8 + d * 2;  // permuted: codes {0,2,4,6}, then {1,3,5,7}
            dot = __builtin_amdgcn_sdot4(static_cast<int>(ce), static_cast<int>(qd[0]), dot, false);
            dot = __builtin_amdgcn_sdot4(static_cast<int>(co), static_cast<int>(qd[1]), dot, false);
        } else {
            const uint32_t *qd = lq + c * 16 + d * 4;
#pragma unroll
            for (int m = 0; m < 4; ++m)
                dot = __builtin_amdgcn_sdot4(
                    static_cast<int>(__builtin_amdgcn_perm(0u, cent[0], (words[d] >> (2 * m)) & 0x03030303u)),
                    static_cast<int>(qd[m]), dot, false);
        }
        constexpr int kPer = S::kCodes / 4;  // codes per dword
        const int pos_end = c * S::kCodes + (d + 1) * kPer;
        const bool closes = GROUP >= S::kCodes ? (d == 3 && pos_end % GROUP == 0) : ((d + 1) * kPer) % GROUP == 0;
        if (closes) {
            const int k = GROUP >= S::kCodes ? 0 : (d + 1) * kPer / GROUP - 1;
            const int g = pos_end / GROUP - 1;
            if (g < groups) {
                if constexpr (DOTS) {
                    if (dots_row) dots_row[g] = dot;
                } else {
                    const float ns = h2f(sl.norm[k]) * cs;  // sdot.cpp:43-44
                    value = value + (static_cast<float>(dot) * ns) * lxs[g];
                }
            }
            dot = 0;
        }
    }
}

template <int KIND, int GROUP, bool DOTS>
__global__ __launch_bounds__(kRowsPerBlock) void sdot_row_kernel(SdotJob job0, const SdotJob *__restrict__ jobs,
                                                                int njobs, SdotGeom geom, int32_t *__restrict__ dots) {
    using S = RowSlot<KIND, GROUP>;
    extern __shared__ __attribute__((aligned(16))) uint32_t row_lds[];
    const int blk = blockIdx.x;
    SdotJob J = job0;
    if (njobs > 0) {
        const ND_CONST SdotJob *cj = (const ND_CONST SdotJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J.codes = cj[j].codes;
        J.norms = cj[j].norms;
        J.q = cj[j].q;
        J.xs = cj[j].xs;
        J.y = cj[j].y;
        J.rows = cj[j].rows;
        J.block_begin = cj[j].block_begin;
    }
    const int tile = blk - J.block_begin;
    const int row = tile * kRowsPerBlock + threadIdx.x;
    const int groups = geom.groups;
    const int dev = geom.windows * kWindow;
    uint32_t *lq = row_lds;
    float *lxs = reinterpret_cast<float *>(row_lds + dev / 4);
    const uint32_t cent[4] = {geom.cent[0], geom.cent[1], geom.cent[2], geom.cent[3]};
    const float cs = geom.centroid_scale;
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms = buffer_rsrc(J.norms + static_cast<size_t>(tile) * groups * kRowsPerBlock,
                                                     static_cast<uint32_t>(groups) * kRowsPerBlock * 2u);
    const int nch = (groups * GROUP + S::kCodes - 1) / S::kCodes;  // chunks holding real positions
    RowSlot<KIND, GROUP> ring[kRowRing];
#pragma unroll
    for (int k = 0; k < kRowRing; ++k) row_load(ring[k], codes, norms, min(k, nch - 1), groups);
    // stage the activation row and its group scales
    const u32x4 *q4 = reinterpret_cast<const u32x4 *>(J.q);
    for (int i = threadIdx.x; i < dev / 16; i += kRowsPerBlock) reinterpret_cast<u32x4 *>(lq)[i] = q4[i];
    for (int i = threadIdx.x; i < groups; i += kRowsPerBlock) lxs[i] = J.xs[i];
    __syncthreads();
    float value = 0.0f;
    int dot = 0;
    int32_t *dots_row = DOTS && row < J.rows ? dots + static_cast<size_t>(row) * groups : nullptr;
    int c0 = 0;
    for (; c0 + kRowRing <= nch; c0 += kRowRing) {
#pragma unroll
        for (int k = 0; k < kRowRing; ++k) {
            row_compute<KIND, GROUP, DOTS>(ring[k], lq, lxs, cent, cs, c0 + k, groups, value, dot, dots_row);
            row_load(ring[k], codes, norms, min(c0 + k + kRowRing, nch - 1), groups);
        }
    }
#pragma unroll
    for (int k = 0; k < kRowRing; ++k)
        if (c0 + k < nch) row_compute<KIND, GROUP, DOTS>(ring[k], lq, lxs, cent, cs, c0 + k, groups, value, dot, dots_row);
    if (!DOTS && row < J.rows) ((ND_GLOBAL float *)J.y)[row] = value;
}

template <int KIND, bool DOTS>
void launch_sdot_row(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks,
                     int32_t *dots, hipStream_t s) {
    const int dev = g.windows * kWindow;
    const size_t lds = static_cast<size_t>(dev) + static_cast<size_t>(g.groups) * 4;
    dim3 grid(blocks), block(kRowsPerBlock);
    switch (g.group) {
    case 8:
        if constexpr (KIND == kNib) {
            hipLaunchKernelGGL((sdot_row_kernel<KIND, 8, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots);
            break;
        }
        [[fallthrough]];
    case 16: hipLaunchKernelGGL((sdot_row_kernel<KIND, 16, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
    case 32: hipLaunchKernelGGL((sdot_row_kernel<KIND, 32, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
    case 64: hipLaunchKernelGGL((sdot_row_kernel<KIND, 64, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
    case 128: hipLaunchKernelGGL((sdot_row_kernel<KIND, 128, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
    default: hipLaunchKernelGGL((sdot_row_kernel<KIND, 256, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
    }
    ND_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// int8 GEMV for batch tiles of 2 .. 16 rows, one thread per output row.
//
// As the row kernel (codes streamed through a register ring, decoded once
// per code dword with v_perm_b32), but the products of a decoded code dword
// with the tile's batch rows run on v_mfma_i32_4x4x4_16b_i8 instead of one
// v_dot4_i32_i8 per batch row: in each of its 16 blocks, block l / 4 of lane
// l, the matrix instruction takes 4 activations of batch row l % 4 (A) and
// the 4 centroids lane l decoded for its own weight row (B), so accumulator
// register r of lane l is the dot of weight row l with batch row r of the
// quad. One quad of batch rows per 4 x 4 x 4 product; NQ quads per tile. The
// tile's permuted int8 activations and group scales are staged in LDS once
// per workgroup; after that barrier the waves never synchronise again. Each
// group closes with the reference's epilogue for every batch row of the tile
//   value += (float(dot) * (half(norm) * cs)) * x_scale[g]
// in group order (sdot.cpp:43-44, 142-149): bit-identical outputs. With
// DOTS the int32 group dots themselves are stored (dots[b][row][g]).
// ---------------------------------------------------------------------------
constexpr int kQuadMaxLds = 160 * 1024;

template <int KIND, int GROUP, int NQ, bool DOTS>
__global__ __launch_bounds__(kRowsPerBlock) void sdot_quad_kernel(SdotJob job0, const SdotJob *__restrict__ jobs,
                                                                 int njobs, SdotGeom geom, int32_t *__restrict__ dots) {
    using S = RowSlot<KIND, GROUP>;
    constexpr int TB = 4 * NQ;  // batch rows of the tile
    extern __shared__ __attribute__((aligned(16))) uint32_t quad_lds[];
    const int blk = blockIdx.x;
    SdotJob J = job0;
    if (njobs > 0) {
        const ND_CONST SdotJob *cj = (const ND_CONST SdotJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J.codes = cj[j].codes;
        J.norms = cj[j].norms;
        J.q = cj[j].q;
        J.xs = cj[j].xs;
        J.y = cj[j].y;
        J.rows = cj[j].rows;
        J.block_begin = cj[j].block_begin;
        J.batch = cj[j].batch;
        J.ystride = cj[j].ystride;
    }
    const int tile = blk - J.block_begin;
    const int row = tile * kRowsPerBlock + threadIdx.x;
    const int groups = geom.groups;
    const int dev = geom.windows * kWindow;
    const int qdw = dev / 4;  // activation dwords per batch row
    const int b0 = static_cast<int>(blockIdx.y) * TB;
    const int nb = min(TB, J.batch - b0);  // valid batch rows of the tile (uniform)
    uint32_t *lq = quad_lds;
    float *lxs = reinterpret_cast<float *>(quad_lds + TB * qdw);
    const uint32_t cent[4] = {geom.cent[0], geom.cent[1], geom.cent[2], geom.cent[3]};
    const float cs = geom.centroid_scale;
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms = buffer_rsrc(J.norms + static_cast<size_t>(tile) * groups * kRowsPerBlock,
                                                     static_cast<uint32_t>(groups) * kRowsPerBlock * 2u);
    const int nch = (groups * GROUP + S::kCodes - 1) / S::kCodes;  // chunks holding real positions
    RowSlot<KIND, GROUP> ring[kRowRing];
#pragma unroll
    for (int k = 0; k < kRowRing; ++k) row_load(ring[k], codes, norms, min(k, nch - 1), groups);
    // stage the tile's activation rows and group scales (rows past the batch as zeros)
    const u32x4 *q4 = reinterpret_cast<const u32x4 *>(J.q) + static_cast<size_t>(b0) * (qdw / 4);
    for (int i = threadIdx.x; i < TB * qdw / 4; i += kRowsPerBlock)
        reinterpret_cast<u32x4 *>(lq)[i] = i / (qdw / 4) < nb ? q4[i] : u32x4{0, 0, 0, 0};
    for (int i = threadIdx.x; i < TB * groups; i += kRowsPerBlock)
        lxs[i] = i / groups < nb ? J.xs[static_cast<size_t>(b0) * groups + i] : 0.0f;
    __syncthreads();
    const int lb = threadIdx.x & 3;  // the batch row of each quad this lane feeds to the matrix instruction
    float value[TB];
#pragma unroll
    for (int b = 0; b < TB; ++b) value[b] = 0.0f;
    v4i acc[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) acc[q] = v4i{0, 0, 0, 0};
    auto chunk = [&](const RowSlot<KIND, GROUP> &sl, int c) {
        constexpr int QPC = KIND == kNib ? 8 : 16;  // activation dwords per chunk
        const uint32_t words[4] = {sl.code.x, sl.code.y, sl.code.z, sl.code.w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t wq[4];  // the centroid dwords of this code dword, in activation-dword order
            constexpr int W = KIND == kNib ? 2 : 4;
            if constexpr (KIND == kNib) {
                decode_nib(words[d], cent[0], cent[1], cent[2], cent[3], wq[0], wq[1]);
            } else {
#pragma unroll
                for (int m = 0; m < 4; ++m) wq[m] = __builtin_amdgcn_perm(0u, cent[0], (words[d] >> (2 * m)) & 0x03030303u);
            }
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const uint32_t *qa = lq + (4 * q + lb) * qdw + c * QPC + d * W;
#pragma unroll
                for (int m = 0; m < W; ++m)
                    acc[q] = __builtin_amdgcn_mfma_i32_4x4x4i8(static_cast<int>(qa[m]), static_cast<int>(wq[m]), acc[q],
                                                              0, 0, 0);
            }
            constexpr int kPer = S::kCodes / 4;  // codes per dword
            const int pos_end = c * S::kCodes + (d + 1) * kPer;
            const bool closes =
                GROUP >= S::kCodes ? (d == 3 && pos_end % GROUP == 0) : ((d + 1) * kPer) % GROUP == 0;
            if (closes) {
                const int k = GROUP >= S::kCodes ? 0 : (d + 1) * kPer / GROUP - 1;
                const int g = pos_end / GROUP - 1;
                if (g < groups) {
                    if constexpr (DOTS) {
                        if (row < J.rows)
#pragma unroll
                            for (int q = 0; q < NQ; ++q)
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    if (4 * q + r < nb)
                                        dots[(static_cast<size_t>(b0 + 4 * q + r) * J.rows + row) * groups + g] =
                                            acc[q][r];
                    } else {
                        const float ns = h2f(sl.norm[k]) * cs;  // sdot.cpp:43-44
#pragma unroll
                        for (int q = 0; q < NQ; ++q)
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                value[4 * q + r] =
                                    value[4 * q + r] + (static_cast<float>(acc[q][r]) * ns) * lxs[(4 * q + r) * groups + g];
                    }
                }
#pragma unroll
                for (int q = 0; q < NQ; ++q) acc[q] = v4i{0, 0, 0, 0};
            }
        }
    };
    int c0 = 0;
    for (; c0 + kRowRing <= nch; c0 += kRowRing) {
#pragma unroll
        for (int k = 0; k < kRowRing; ++k) {
            chunk(ring[k], c0 + k);
            row_load(ring[k], codes, norms, min(c0 + k + kRowRing, nch - 1), groups);
        }
    }
#pragma unroll
    for (int k = 0; k < kRowRing; ++k)
        if (c0 + k < nch) chunk(ring[k], c0 + k);
    if constexpr (!DOTS) {
        if (row < J.rows) {
#pragma unroll
            for (int b = 0; b < TB; ++b)
                if (b < nb) ((ND_GLOBAL float *)J.y)[static_cast<size_t>(b0 + b) * (J.ystride ? J.ystride : J.rows) + row] = value[b];
        }
    }
}

template <int KIND, bool DOTS>
bool launch_sdot_quad(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int batch,
                      int32_t *dots, hipStream_t s) {
    const int dev = g.windows * kWindow;
    const int tb = batch >= 16 ? 16 : (batch + 3) / 4 * 4;  // rows per tile
    const size_t lds = static_cast<size_t>(tb) * dev + static_cast<size_t>(tb) * g.groups * 4;
    if (lds > kQuadMaxLds || g.group > kWindow) return false;
    dim3 grid(blocks, (batch + tb - 1) / tb), block(kRowsPerBlock);
    auto go = [&](auto nq) {
        constexpr int NQ = decltype(nq)::value;
        switch (g.group) {
        case 8:
            if constexpr (KIND == kNib) {
                hipLaunchKernelGGL((sdot_quad_kernel<KIND, 8, NQ, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots);
                break;
            }
            [[fallthrough]];
        case 16: hipLaunchKernelGGL((sdot_quad_kernel<KIND, 16, NQ, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
        case 32: hipLaunchKernelGGL((sdot_quad_kernel<KIND, 32, NQ, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
        case 64: hipLaunchKernelGGL((sdot_quad_kernel<KIND, 64, NQ, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
        case 128: hipLaunchKernelGGL((sdot_quad_kernel<KIND, 128, NQ, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
        default: hipLaunchKernelGGL((sdot_quad_kernel<KIND, 256, NQ, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
        }
    };
    switch (tb / 4) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 3: go(std::integral_constant<int, 3>{}); break;
    default: go(std::integral_constant<int, 4>{}); break;
    }
    ND_HIP(hipGetLastError());
    return true;
}

// ---------------------------------------------------------------------------
// int8 GEMV for batch tiles of 16 rows, groups of one or more whole code
// chunks (4-bit: 32 .. 256, 2-bit: 64 .. 256), one wave per 64 weight rows.
//
// Each code chunk (16 bytes per weight row: 32 four-bit or 64 two-bit codes)
// is 4 (4-bit) or 8 (2-bit) v_mfma_i32_16x16x32_i8, 1 or 2 per 16 of the
// wave's weight rows: lane (j, t) = (l % 16, l / 16) decodes code dword t of
// weight row 16 m + j for each m (every code decoded once) as the B operand,
// and feeds the permuted activations of batch row j that pair with that dword
// (A, one LDS read per chunk for all its products); accumulator register r of
// lane (j, t) is then the dot of weight row 16 m + j with batch row 4 t + r. The
// tile's activations and group scales are staged in LDS once per workgroup.
// Each group closes with the reference's epilogue for every batch row
//   value += (float(dot) * (half(norm) * cs)) * x_scale[g]
// in group order (sdot.cpp:43-44, 142-149): bit-identical outputs. With DOTS
// the int32 group dots are stored (dots[b][row][g]).
// ---------------------------------------------------------------------------
struct Tile16Slot {
    uint32_t code[4];  // dword t of the chunk, weight rows 16 m + j
    uint16_t norm[4];  // their group norms, loaded with the chunk that closes a group
};

template <int KIND, int GROUP, bool DOTS>
__global__ __launch_bounds__(kRowsPerBlock) void sdot_tile16_kernel(SdotJob job0, const SdotJob *__restrict__ jobs,
                                                                   int njobs, SdotGeom geom, int32_t *__restrict__ dots) {
    constexpr int CODES = KIND == kNib ? 32 : 64;  // codes per chunk
    constexpr int H = CODES / 32;                  // products per chunk and 16 weight rows
    static_assert(GROUP >= CODES && GROUP <= kWindow, "one or more whole chunks per group");
    constexpr int TB = 16;
    constexpr int CPG = GROUP / CODES;  // chunks per group (divides kRowRing)
    static_assert(kRowRing % CPG == 0, "group closes at fixed ring slots");
    extern __shared__ __attribute__((aligned(16))) uint32_t t16_lds[];
    const int blk = blockIdx.x;
    SdotJob J = job0;
    if (njobs > 0) {
        const ND_CONST SdotJob *cj = (const ND_CONST SdotJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J.codes = cj[j].codes;
        J.norms = cj[j].norms;
        J.q = cj[j].q;
        J.xs = cj[j].xs;
        J.y = cj[j].y;
        J.rows = cj[j].rows;
        J.block_begin = cj[j].block_begin;
        J.batch = cj[j].batch;
        J.ystride = cj[j].ystride;
    }
    const int tile = blk - J.block_begin;
    const int lane = threadIdx.x & 63;
    const int jr = lane & 15, t = lane >> 4;
    const int wrow = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * 64;  // the wave's first row in the tile
    const int groups = geom.groups;
    const int dev = geom.windows * kWindow;
    const int qdw = dev / 4;
    const int b0 = static_cast<int>(blockIdx.y) * TB;
    const int nb = min(TB, J.batch - b0);
    uint32_t *lq = t16_lds;
    float *lxs = reinterpret_cast<float *>(t16_lds + TB * qdw);
    const uint32_t cent[4] = {geom.cent[0], geom.cent[1], geom.cent[2], geom.cent[3]};
    const float cs = geom.centroid_scale;
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms = buffer_rsrc(J.norms + static_cast<size_t>(tile) * groups * kRowsPerBlock,
                                                     static_cast<uint32_t>(groups) * kRowsPerBlock * 2u);
    const int nch = groups * CPG;  // chunks holding real positions
    // per-lane offsets: code dword t of weight row wrow + 16 m + jr, and its fp16 norm
    uint32_t cv[4], nv[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        cv[m] = (wrow + 16 * m + jr) * 16u + 4u * t;
        nv[m] = (wrow + 16 * m + jr) * 2u;
    }
    // The ring prefetch past the last chunk re-reads the last chunk (never used).
    auto load = [&](Tile16Slot &sl, int c, bool closes) {
        const int so = __builtin_amdgcn_readfirstlane(c * kRowsPerBlock * 16);
#pragma unroll
        for (int m = 0; m < 4; ++m) sl.code[m] = __builtin_amdgcn_raw_buffer_load_b32(codes, cv[m], so, kStreamLoad);
        if (closes) {
            const int no = __builtin_amdgcn_readfirstlane(c / CPG * kRowsPerBlock * 2);
#pragma unroll
            for (int m = 0; m < 4; ++m) sl.norm[m] = __builtin_amdgcn_raw_buffer_load_b16(norms, nv[m], no, 0);
        }
    };
    Tile16Slot ring[kRowRing];
#pragma unroll
    for (int k = 0; k < kRowRing; ++k) load(ring[k], min(k, nch - 1), (k + 1) % CPG == 0);
    // stage the tile's activation rows and group scales (rows past the batch as zeros)
    const u32x4 *q4 = reinterpret_cast<const u32x4 *>(J.q) + static_cast<size_t>(b0) * (qdw / 4);
    for (int i = threadIdx.x; i < TB * qdw / 4; i += kRowsPerBlock)
        reinterpret_cast<u32x4 *>(lq)[i] = i / (qdw / 4) < nb ? q4[i] : u32x4{0, 0, 0, 0};
    for (int i = threadIdx.x; i < TB * groups; i += kRowsPerBlock)
        lxs[i] = i / groups < nb ? J.xs[static_cast<size_t>(b0) * groups + i] : 0.0f;
    __syncthreads();
    float value[4][4];  // [m][r]: weight row wrow + 16 m + jr, batch row 4 t + r
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) value[m][r] = 0.0f;
    v4i acc[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[m] = v4i{0, 0, 0, 0};
    const uint32_t *qrow = lq + jr * qdw + 2 * H * t;  // batch row jr: the activation dwords of code dword t
    const float *xrow = lxs + 4 * t * groups;      // scales of batch rows 4t .. 4t + 3
    auto chunk = [&](const Tile16Slot &sl, int c, bool closes) {
        long a[H];
        if constexpr (KIND == kNib) {
            const auto q2 = *reinterpret_cast<const uint32_t __attribute__((ext_vector_type(2))) *>(qrow + c * 8);
            a[0] = static_cast<long>(q2[0]) | (static_cast<long>(q2[1]) << 32);
        } else {
            const u32x4 q4v = *reinterpret_cast<const u32x4 *>(qrow + c * 16);
            a[0] = static_cast<long>(q4v.x) | (static_cast<long>(q4v.y) << 32);
            a[1] = static_cast<long>(q4v.z) | (static_cast<long>(q4v.w) << 32);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            uint32_t wq[2 * H];  // the centroid dwords of code dword t, in activation-dword order
            if constexpr (KIND == kNib) {
                decode_nib(sl.code[m], cent[0], cent[1], cent[2], cent[3], wq[0], wq[1]);
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    wq[k] = __builtin_amdgcn_perm(0u, cent[0], (sl.code[m] >> (2 * k)) & 0x03030303u);
            }
#pragma unroll
            for (int h = 0; h < H; ++h) {
                const long b = static_cast<long>(wq[2 * h]) | (static_cast<long>(wq[2 * h + 1]) << 32);
                acc[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[h], b, acc[m], 0, 0, 0);
            }
        }
        if (closes) {
            const int g = c / CPG;
            if constexpr (DOTS) {
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const int row = tile * kRowsPerBlock + wrow + 16 * m + jr;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (4 * t + r < nb && row < J.rows)
                            dots[(static_cast<size_t>(b0 + 4 * t + r) * J.rows + row) * groups + g] = acc[m][r];
                }
            } else {
                float xsb[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) xsb[r] = xrow[r * groups + g];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const float ns = h2f(sl.norm[m]) * cs;  // sdot.cpp:43-44
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        value[m][r] = value[m][r] + (static_cast<float>(acc[m][r]) * ns) * xsb[r];
                }
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) acc[m] = v4i{0, 0, 0, 0};
        }
    };
    int c0 = 0;
    for (; c0 + kRowRing <= nch; c0 += kRowRing) {
#pragma unroll
        for (int k = 0; k < kRowRing; ++k) {
            chunk(ring[k], c0 + k, (k + 1) % CPG == 0);
            load(ring[k], min(c0 + k + kRowRing, nch - 1), (k + 1) % CPG == 0);
        }
    }
#pragma unroll
    for (int k = 0; k < kRowRing; ++k)
        if (c0 + k < nch) chunk(ring[k], c0 + k, (k + 1) % CPG == 0);
    if constexpr (!DOTS) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int row = tile * kRowsPerBlock + wrow + 16 * m + jr;
            if (row < J.rows)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (4 * t + r < nb)
                        ((ND_GLOBAL float *)J.y)[static_cast<size_t>(b0 + 4 * t + r) * (J.ystride ? J.ystride : J.rows) + row] = value[m][r];
        }
    }
}

template <int KIND, bool DOTS>
bool launch_sdot_tile16(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int batch,
                        int32_t *dots, hipStream_t s) {
    const int dev = g.windows * kWindow;
    const size_t lds = static_cast<size_t>(16) * dev + static_cast<size_t>(16) * g.groups * 4;
    if (g.group < (KIND == kNib ? 32 : 64) || g.group > kWindow || lds > kQuadMaxLds) return false;
    dim3 grid(blocks, (batch + 15) / 16), block(kRowsPerBlock);
    switch (g.group) {
    case 32:
        if constexpr (KIND == kNib) {
            hipLaunchKernelGGL((sdot_tile16_kernel<KIND, 32, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots);
            break;
        }
        [[fallthrough]];
    case 64: hipLaunchKernelGGL((sdot_tile16_kernel<KIND, 64, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
    case 128: hipLaunchKernelGGL((sdot_tile16_kernel<KIND, 128, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
    default: hipLaunchKernelGGL((sdot_tile16_kernel<KIND, 256, DOTS>), grid, block, lds, s, job0, jobs, njobs, g, dots); break;
    }
    ND_HIP(hipGetLastError());
    return true;
}

// ---------------------------------------------------------------------------
// int8 MFMA path split over K, for small matrices (decode layers, any batch)
//
// A workgroup of KS waves (8, or 16 from 64 groups: ks_waves) shares one
// (32 weight rows, 32 batch rows) tile; wave w takes groups w, w + KS, ...
// Each round every wave turns its group's int32 accumulator into the
// reference's terms (float(dot) * ns) * x_scale (sdot.cpp:142-149) and parks
// them in LDS (double-buffered by round); after one barrier, the owner of
// each accumulator register adds the KS terms in group order. Each output is
// therefore value += term_g for g = 0, 1, 2, ... exactly as the reference
// sums, and many more waves cover a small matrix.
// ---------------------------------------------------------------------------

template <int KIND, int GROUP, int J>
__device__ __forceinline__ void mfma_terms(const MfmaSlot<KIND, GROUP, J> &sl, const uint32_t cent[4], float cs,
                                           float (&term)[4 * J]) {
    float value[4 * J];
#pragma unroll
    for (int r = 0; r < 4 * J; ++r) value[r] = -0.0f;  // -0 + t == t exactly, so value ends as the term
    mfma_group(sl, cent, cs, value);
#pragma unroll
    for (int r = 0; r < 4 * J; ++r) term[r] = value[r];
}

// XIN (batch 1): the workgroup prepares the job's input row J.x into LDS
// first, each wave the groups its rounds read (prepare_lane /
// prepare_group_wave: the prepare kernels' arithmetic), so the plan launches
// no prepare kernel; the outputs are the same bits.
template <int KIND, int GROUP, int J, bool XIN, int KS>
__global__ __launch_bounds__(KS * 64) void sdot_mfma_ks_kernel(SdotJob job0, const SdotJob *__restrict__ jobs,
                                                                int njobs, SdotGeom geom) {
    constexpr int R = 4 * J;                          // accumulator registers in use
    constexpr int kOwn = (R + KS - 1) / KS;         // registers each wave sums
    __shared__ float park[2][KS][R][64];
    extern __shared__ __attribute__((aligned(16))) uint8_t xin_lds[];  // XIN: q [dev], then scales [groups]
    const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int rb = blockIdx.x;                        // 32-row block across the plan
    const int blk = rb / (kRowsPerBlock / 32);
    SdotJob J0 = job0;
    if (njobs > 0) {
        const ND_CONST SdotJob *cj = (const ND_CONST SdotJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J0.codes = cj[j].codes;
        J0.norms = cj[j].norms;
        J0.q = cj[j].q;
        J0.y = cj[j].y;
        J0.rows = cj[j].rows;
        J0.block_begin = cj[j].block_begin;
        J0.batch = cj[j].batch;
        J0.ystride = cj[j].ystride;
        J0.xst = cj[j].xst;
        J0.x = cj[j].x;
    }
    const int rows = J0.rows, batch = J0.batch;
    const int tile = blk - J0.block_begin;
    const int rt = (rb % (kRowsPerBlock / 32)) * 32 + i;
    const int row = tile * kRowsPerBlock + rt;
    const int b0 = static_cast<int>(blockIdx.y) * 32;
    const int groups = geom.groups;
    const int dev = geom.windows * kWindow;
    const uint32_t cent[4] = {geom.cent[0], geom.cent[1], geom.cent[2], geom.cent[3]};
    const float cs = geom.centroid_scale;
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J0.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms = buffer_rsrc(J0.norms + static_cast<size_t>(tile) * groups * kRowsPerBlock,
                                                     static_cast<uint32_t>(groups) * kRowsPerBlock * 2u);
    const int tile_rows = min(32, batch - b0);
    const __amdgpu_buffer_rsrc_t q =
        buffer_rsrc(reinterpret_cast<const int8_t *>(J0.q) + static_cast<size_t>(b0) * dev,
                    static_cast<uint32_t>(tile_rows) * dev);
    const __amdgpu_buffer_rsrc_t xst = buffer_rsrc(J0.xst, static_cast<uint32_t>(groups) * batch * 4u);

    int8_t *qst = reinterpret_cast<int8_t *>(xin_lds);
    float *scst = reinterpret_cast<float *>(xin_lds + dev);
    if constexpr (XIN) {
        const float *xv = J0.x;
        const int in = geom.in, padded = geom.padded;
        if constexpr (GROUP <= 64) {  // 64 / GROUP of the wave's groups per pass, one lane per position
            constexpr int PER = 64 / GROUP;
            for (int k = 0; w + KS * PER * k < groups; ++k) {
                const int g = w + KS * (PER * k + lane / GROUP);
                const int p = g * GROUP + lane % GROUP;
                const float r = p < in ? xv[p] : 0.0f;
                prepare_lane<GROUP>(r, lane, p, padded, dev, geom.scale, KIND, qst, scst + (g < groups ? g : 0),
                                    nullptr);
            }
        } else {
            for (int g = w; g < groups; g += KS) {
                float r[GROUP / 64];
#pragma unroll
                for (int k = 0; k < GROUP / 64; ++k) {
                    const int p = g * GROUP + lane + 64 * k;
                    r[k] = p < in ? xv[p] : 0.0f;
                }
                prepare_group_wave<GROUP>(r, lane, g * GROUP, padded, dev, geom.scale, KIND, qst, scst + g, nullptr);
            }
        }
        __syncthreads();
    }
    auto load = [&](MfmaSlot<KIND, GROUP, J> &sl, int g) {
        if constexpr (XIN) mfma_load_x(sl, codes, norms, qst, scst, g, rt, i, h, dev, groups);
        else mfma_load(sl, codes, norms, q, xst, g, rt, i, h, dev, batch, b0);
    };

    float value[kOwn];
#pragma unroll
    for (int k = 0; k < kOwn; ++k) value[k] = 0.0f;
    const int rounds = (groups + KS - 1) / KS;
    MfmaSlot<KIND, GROUP, J> cur, nxt;
    load(cur, w);
    for (int r = 0; r < rounds; ++r) {
        // next round's group (past the last group: zeros, or data that is never used)
        load(nxt, (r + 1) * KS + w);
        float term[R];
        mfma_terms(cur, cent, cs, term);
#pragma unroll
        for (int k = 0; k < R; ++k) park[r & 1][w][k][lane] = term[k];
        __syncthreads();
        const int live = min(KS, groups - r * KS);  // groups of this round (uniform)
#pragma unroll
        for (int k = 0; k < kOwn; ++k) {
            const int reg = w + k * KS;
            if (reg < R)
                for (int src = 0; src < live; ++src) value[k] = value[k] + park[r & 1][src][reg][lane];
        }
        cur = nxt;
    }
    if (row < rows) {
#pragma unroll
        for (int k = 0; k < kOwn; ++k) {
            const int reg = w + k * KS;
            if (reg >= R) continue;
            const int m = b0 + 8 * (reg / 4) + 4 * h + (reg % 4);
            if (m < batch) ((ND_GLOBAL float *)J0.y)[static_cast<size_t>(m) * (J0.ystride ? J0.ystride : rows) + row] = value[k];
        }
    }
}

template <int KIND, int J, bool XIN, int KS>
void launch_sdot_ks_waves(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int batch,
                          hipStream_t s) {
    dim3 grid(blocks * (kRowsPerBlock / 32), (batch + 31) / 32), block(KS * 64);
    const size_t lds = XIN ? static_cast<size_t>(g.windows) * kWindow + static_cast<size_t>(g.groups) * 4 : 0;
    switch (g.group) {
    case 32: hipLaunchKernelGGL((sdot_mfma_ks_kernel<KIND, 32, J, XIN, KS>), grid, block, lds, s, job0, jobs, njobs, g); break;
    case 64: hipLaunchKernelGGL((sdot_mfma_ks_kernel<KIND, 64, J, XIN, KS>), grid, block, lds, s, job0, jobs, njobs, g); break;
    case 128: hipLaunchKernelGGL((sdot_mfma_ks_kernel<KIND, 128, J, XIN, KS>), grid, block, lds, s, job0, jobs, njobs, g); break;
    default: hipLaunchKernelGGL((sdot_mfma_ks_kernel<KIND, 256, J, XIN, KS>), grid, block, lds, s, job0, jobs, njobs, g); break;
    }
    ND_HIP(hipGetLastError());
}

// 16 waves per workgroup from 64 groups (half the rounds), as the 16 x 16 K
// split does; NEEDLE2_GPU_INT8_KS16_WAVES = 8 / 16 overrides both.
static int ks_waves(const SdotGeom &g) {
    const char *mode = std::getenv("NEEDLE2_GPU_INT8_KS16_WAVES");
    if (mode && std::strcmp(mode, "8") == 0) return 8;
    if (mode && std::strcmp(mode, "16") == 0) return 16;
    return g.groups >= 64 ? 16 : 8;
}

template <int KIND, int J, bool XIN = false>
void launch_sdot_ks_j(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int batch,
                      hipStream_t s) {
    if (ks_waves(g) == 16) launch_sdot_ks_waves<KIND, J, XIN, 16>(g, job0, jobs, njobs, blocks, batch, s);
    else launch_sdot_ks_waves<KIND, J, XIN, 8>(g, job0, jobs, njobs, blocks, batch, s);
}

template <int KIND>
void launch_sdot_ks(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int batch,
                    hipStream_t s) {
    if (batch <= 8) launch_sdot_ks_j<KIND, 1>(g, job0, jobs, njobs, blocks, batch, s);
    else if (batch <= 16) launch_sdot_ks_j<KIND, 2>(g, job0, jobs, njobs, blocks, batch, s);
    else launch_sdot_ks_j<KIND, 4>(g, job0, jobs, njobs, blocks, batch, s);
}

// ---------------------------------------------------------------------------
// int8 path split over K on 16 x 16 tiles, for small matrices (decode-layer
// projections and prompt chunks at batch 2 and more)
//
// As sdot_mfma_ks_kernel, with a workgroup of KS (8, or 16 from 64 groups)
// waves sharing one tile of 16 weight rows x 16 batch rows, so a small matrix
// spreads over four times the workgroups. Wave w takes groups w, w + KS, ...;
// each 32-position step of a group is one v_mfma_i32_16x16x32_i8: lane
// (j, t) = (l % 16, l / 16)
// feeds batch row j's activations of positions 8t .. 8t + 7 of the step (A)
// and weight row j's decoded centroids of the same positions (B): code
// dword t of the step's 32 four-bit codes, or crumb selectors 2(t % 2) and
// 2(t % 2) + 1 of code dword t / 2 of its 32 two-bit codes; accumulator
// register r of lane (j, t) is then the dot of weight row j with batch row
// 4 t + r. Each round every wave turns its group's four dots into the
// reference's terms (float(dot) * ns) * x_scale (sdot.cpp:142-149) and parks
// them in LDS; after one barrier wave r (< 4) adds register r's KS terms in
// group order, so every output is value += term_g for g = 0, 1, 2, ... as
// the reference sums: bit-identical outputs.
//
// MB = 2 (PREP): a workgroup takes 32 weight rows (two 16-row blocks, every
// wave two MFMA chains sharing the activation operand) and, with PREP, turns
// its 32 outputs of each batch row - one whole group of 32 positions of the
// next projection's input - into that projection's prepared input as the
// prepare kernel would from the stored outputs (prepare_lane: FWHT, absmax,
// quantiser; same bits), so the next plan launches no prepare kernel.
// ---------------------------------------------------------------------------
template <int GROUP, int MB>
struct Ks16Slot {
    static constexpr int kSteps = GROUP / 32;
    uint32_t code[MB][kSteps];  // per row block: the code dword of each step holding positions 8t .. 8t + 7, weight row j
    uint32_t q[2 * kSteps];     // batch row j's activation dwords 2t, 2t + 1 of each step
    float xs[4];                // scales of batch rows 4t .. 4t + 3
    uint16_t norm[MB];          // weight row j's group norm, per row block
};

template <int KIND, int GROUP, int MB, bool PREP, int KS>
__global__ __launch_bounds__(KS * 64) void sdot_ks16_kernel(SdotJob job0, const SdotJob *__restrict__ jobs,
                                                             int njobs, SdotGeom geom, PrepOut po) {
    static_assert(MB == 1 || MB == 2, "one or two 16-row blocks");
    static_assert(!PREP || MB == 2, "the prepared groups are 32 outputs");
    using S = Ks16Slot<GROUP, MB>;
    constexpr int RB = 16 * MB;  // weight rows per workgroup
    __shared__ float park[2][KS][4 * MB][64];
    const int lane = threadIdx.x & 63, jr = lane & 15, t = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int rb = blockIdx.x;  // RB-row block across the plan
    const int blk = rb / (kRowsPerBlock / RB);
    SdotJob J0 = job0;
    if (njobs > 0) {
        const ND_CONST SdotJob *cj = (const ND_CONST SdotJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J0.codes = cj[j].codes;
        J0.norms = cj[j].norms;
        J0.q = cj[j].q;
        J0.y = cj[j].y;
        J0.rows = cj[j].rows;
        J0.block_begin = cj[j].block_begin;
        J0.batch = cj[j].batch;
        J0.ystride = cj[j].ystride;
        J0.xst = cj[j].xst;
    }
    const int rows = J0.rows, batch = J0.batch;
    const int tile = blk - J0.block_begin;
    const int rbase = (rb % (kRowsPerBlock / RB)) * RB;  // the workgroup's first weight row within the tile
    const int b0 = static_cast<int>(blockIdx.y) * 16;
    const int nb = min(16, batch - b0);
    const int groups = geom.groups;
    const int dev = geom.windows * kWindow;
    const uint32_t cent[4] = {geom.cent[0], geom.cent[1], geom.cent[2], geom.cent[3]};
    const float cs = geom.centroid_scale;
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J0.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms = buffer_rsrc(J0.norms + static_cast<size_t>(tile) * groups * kRowsPerBlock,
                                                     static_cast<uint32_t>(groups) * kRowsPerBlock * 2u);
    // batch rows past the tile's last read zeros (their offsets lie past the resource's end)
    const __amdgpu_buffer_rsrc_t q = buffer_rsrc(reinterpret_cast<const int8_t *>(J0.q) + static_cast<size_t>(b0) * dev,
                                                 static_cast<uint32_t>(nb) * dev);
    const __amdgpu_buffer_rsrc_t xst = buffer_rsrc(J0.xst, static_cast<uint32_t>(groups) * batch * 4u);
    // code byte offset of this lane's dword within a 16-byte chunk (4-bit: one step per chunk; 2-bit: the
    // step's half of a 64-position chunk is added per step), per row block
    const uint32_t qv = static_cast<uint32_t>(jr) * dev + 8u * t;
    uint32_t cv[MB], nv[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
        const int rt = rbase + 16 * m + jr;
        cv[m] = rt * 16u + (KIND == kNib ? 4u * t : 4u * (t >> 1));
        nv[m] = rt * 2u;
    }
    auto load = [&](S &sl, int g) {  // g < groups
#pragma unroll
        for (int st = 0; st < S::kSteps; ++st) {
            const int c = g * S::kSteps + st;  // step of 32 positions
            const int so = KIND == kNib ? c * kRowsPerBlock * 16 : (c >> 1) * kRowsPerBlock * 16 + (c & 1) * 8;
#pragma unroll
            for (int m = 0; m < MB; ++m)
                sl.code[m][st] = __builtin_amdgcn_raw_buffer_load_b32(codes, cv[m], __builtin_amdgcn_readfirstlane(so), 0);
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(q, qv + c * 32u, 0, 0);
            sl.q[2 * st] = v[0];
            sl.q[2 * st + 1] = v[1];
        }
        // scales of batch rows b0 + 4t .. + 3 (rows past the batch read the last row's, never stored)
        const int so = __builtin_amdgcn_readfirstlane(g * batch * 4);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            sl.xs[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xst, min(b0 + 4 * t + k, batch - 1) * 4u, so, 0));
#pragma unroll
        for (int m = 0; m < MB; ++m)
            sl.norm[m] = __builtin_amdgcn_raw_buffer_load_b16(norms, nv[m], __builtin_amdgcn_readfirstlane(g * kRowsPerBlock * 2), 0);
    };
    // wave w < 4 MB sums accumulator register w % 4 of row block w / 4: batch row 4t + w % 4, weight row
    // rbase + 16 (w / 4) + jr
    float value = 0.0f;
    const int rounds = (groups + KS - 1) / KS;
    S cur, nxt;
    load(cur, min(w, groups - 1));
    for (int r = 0; r < rounds; ++r) {
        load(nxt, min((r + 1) * KS + w, groups - 1));  // past the last group: re-read, never used
        v4i acc[MB];
#pragma unroll
        for (int m = 0; m < MB; ++m) acc[m] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int st = 0; st < S::kSteps; ++st) {
            const long a = static_cast<long>(cur.q[2 * st]) | (static_cast<long>(cur.q[2 * st + 1]) << 32);
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                uint32_t ce, co;
                if constexpr (KIND == kNib) {
                    decode_nib(cur.code[m][st], cent[0], cent[1], cent[2], cent[3], ce, co);
                } else {  // crumb selectors 2 (t % 2) and 2 (t % 2) + 1 of the dword
                    const uint32_t wd = cur.code[m][st] >> (4 * (t & 1));
                    ce = __builtin_amdgcn_perm(0u, cent[0], wd & 0x03030303u);
                    co = __builtin_amdgcn_perm(0u, cent[0], (wd >> 2) & 0x03030303u);
                }
                const long b = static_cast<long>(ce) | (static_cast<long>(co) << 32);
                acc[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, acc[m], 0, 0, 0);
            }
        }
#pragma unroll
        for (int m = 0; m < MB; ++m) {
            const float ns = h2f(cur.norm[m]) * cs;  // sdot.cpp:43-44
#pragma unroll
            for (int k = 0; k < 4; ++k) park[r & 1][w][4 * m + k][lane] = (static_cast<float>(acc[m][k]) * ns) * cur.xs[k];
        }
        __syncthreads();
        const int live = min(KS, groups - r * KS);  // groups of this round (uniform)
        if (w < 4 * MB)
            for (int src = 0; src < live; ++src) value = value + park[r & 1][src][w][lane];
        cur = nxt;
    }
    const int row = tile * kRowsPerBlock + rbase + 16 * (w / 4) + jr;
    const int m = b0 + 4 * t + (w % 4);
    if (w < 4 * MB && row < rows && m < batch)
        ((ND_GLOBAL float *)J0.y)[static_cast<size_t>(m) * (J0.ystride ? J0.ystride : rows) + row] = value;
    if constexpr (PREP) {
        // the 16 x 32 outputs through LDS (rows past the matrix as the zeros the prepare kernel pads with),
        // then wave w prepares batch rows 2w (lanes 0-31) and 2w + 1 (lanes 32-63) of the group
        __shared__ float yl[16][33];
        if (w < 8) yl[4 * t + (w % 4)][16 * (w / 4) + jr] = row < rows ? value : 0.0f;
        __syncthreads();
        if (w < 8) {
            const int bl = 2 * w + (lane >> 5), pos = lane & 31;
            const int b = b0 + bl;
            const int p = tile * kRowsPerBlock + rbase + pos;  // position in the next projection's input row
            const int gi = p / 32;
            const size_t bs = static_cast<size_t>(b < batch ? b : 0);
            prepare_lane<32>(yl[bl][pos], lane, p, po.padded, po.dev, po.scale, po.kind, po.q + bs * po.dev,
                             po.xs + bs * po.groups + gi, po.xst + static_cast<size_t>(gi) * po.batch + bs, b < batch);
        }
    }
}

template <int KIND, int MB, bool PREP, int KS>
void launch_sdot_ks16_waves(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks,
                            int batch, const PrepOut &po, hipStream_t s) {
    dim3 grid(blocks * (kRowsPerBlock / (16 * MB)), (batch + 15) / 16), block(KS * 64);
    switch (g.group) {
    case 32: hipLaunchKernelGGL((sdot_ks16_kernel<KIND, 32, MB, PREP, KS>), grid, block, 0, s, job0, jobs, njobs, g, po); break;
    case 64: hipLaunchKernelGGL((sdot_ks16_kernel<KIND, 64, MB, PREP, KS>), grid, block, 0, s, job0, jobs, njobs, g, po); break;
    case 128: hipLaunchKernelGGL((sdot_ks16_kernel<KIND, 128, MB, PREP, KS>), grid, block, 0, s, job0, jobs, njobs, g, po); break;
    default: hipLaunchKernelGGL((sdot_ks16_kernel<KIND, 256, MB, PREP, KS>), grid, block, 0, s, job0, jobs, njobs, g, po); break;
    }
    ND_HIP(hipGetLastError());
}

// 16 waves per workgroup (one group each per round) from 64 groups: half
// the rounds of 8 waves, each round's terms still summed in group order
// (decode-layer down projection, K = 2048: 7.2 -> 6.7 us; with 16 groups the
// larger workgroups measured slower, 5.2 -> 6.0 us); ks_waves.
static int ks16_waves(const SdotGeom &g) { return ks_waves(g); }

template <int KIND, int MB, bool PREP>
void launch_sdot_ks16_kind(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks,
                           int batch, const PrepOut &po, hipStream_t s) {
    if (ks16_waves(g) == 16) launch_sdot_ks16_waves<KIND, MB, PREP, 16>(g, job0, jobs, njobs, blocks, batch, po, s);
    else launch_sdot_ks16_waves<KIND, MB, PREP, 8>(g, job0, jobs, njobs, blocks, batch, po, s);
}

// 32-row workgroups (two MFMA chains per wave) from 4 row tiles and 16
// groups: fewer, fuller workgroups for the larger decode projections (Q|K|V
// 1536 x 512 g32 at 64 sequences: 5.2 -> 4.8 us); otherwise the 16-row form
// keeps more workgroups (a 512 x 2048 down projection: 6.7 vs 7.8 us; a
// 32-token chunk's 1536 x 512 g128 projection, 4 groups: engine prefill
// 27.3-27.8 K vs 26.9-27.0 K tokens/s). NEEDLE2_GPU_INT8_KS16_ROWS = 16 / 32
// overrides.
static int ks16_rows(const SdotGeom &g, int blocks) {
    const char *mode = std::getenv("NEEDLE2_GPU_INT8_KS16_ROWS");
    if (mode && std::strcmp(mode, "16") == 0) return 16;
    if (mode && std::strcmp(mode, "32") == 0) return 32;
    return blocks >= 4 && g.groups >= 16 ? 32 : 16;
}

bool launch_sdot_ks16(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int batch,
                      hipStream_t s) {
    if (g.group < 32 || g.group > kWindow) return false;
    const PrepOut none{};
    if (ks16_rows(g, blocks) == 32) {
        if (g.kind == kNib) launch_sdot_ks16_kind<kNib, 2, false>(g, job0, jobs, njobs, blocks, batch, none, s);
        else launch_sdot_ks16_kind<kCrumb, 2, false>(g, job0, jobs, njobs, blocks, batch, none, s);
    } else {
        if (g.kind == kNib) launch_sdot_ks16_kind<kNib, 1, false>(g, job0, jobs, njobs, blocks, batch, none, s);
        else launch_sdot_ks16_kind<kCrumb, 1, false>(g, job0, jobs, njobs, blocks, batch, none, s);
    }
    return true;
}

int device_cus() {
    static int cus = [] {
        int dev = 0, n = 256;
        if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        return n;
    }();
    return cus;
}

// The batch is covered by tiles of 16, 8, 4, 2 and 1 rows (largest first),
// one tile per blockIdx.y. A tile size that would leave fewer than two
// workgroups per CU is skipped: small matrices with many batch rows (a
// decode batch) trade decode reuse for parallelism.
template <int KIND>
void launch_sdot_kind(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int batch,
                      hipStream_t s) {
    int b = 0;
    const int want = 2 * device_cus();
    auto run = [&](int bt, auto launcher) {
        const int n = (batch - b) / bt * bt;
        if (n <= 0) return;
        if (bt > 1 && static_cast<long>(blocks) * (n / bt) < want) return;
        launcher(b, b + n);
        b += n;
    };
    run(16, [&](int b0, int b1) { launch_sdot_bt<KIND, 16>(g, job0, jobs, njobs, blocks, b0, b1, s); });
    run(8, [&](int b0, int b1) { launch_sdot_bt<KIND, 8>(g, job0, jobs, njobs, blocks, b0, b1, s); });
    run(4, [&](int b0, int b1) { launch_sdot_bt<KIND, 4>(g, job0, jobs, njobs, blocks, b0, b1, s); });
    run(2, [&](int b0, int b1) { launch_sdot_bt<KIND, 2>(g, job0, jobs, njobs, blocks, b0, b1, s); });
    run(1, [&](int b0, int b1) { launch_sdot_bt<KIND, 1>(g, job0, jobs, njobs, blocks, b0, b1, s); });
}

// Prepare for groups of 8 .. 64 positions, one pass without LDS: lane t of
// block (segment, vector) owns position 256 * segment + t; the group FWHT
// runs as in-wave butterflies (the reference's stage order and operands),
// the group absmax as an in-wave max, then the reference's quantiser
// (sdot.cpp:56-81: scale = absmax / 127, 1 for an all-zero group, absmax if
// the quotient underflows; q = clamp(rint(x / scale), +-127) with IEEE
// division), stored in the permuted order the GEMV decode expects. Same
// values as sdot_prepare_kernel, bit for bit.
template <int GROUP>
__global__ __launch_bounds__(256) void sdot_prepare_wave_kernel(const float *__restrict__ x0,
                                                                const float *const *__restrict__ xptr, int batch,
                                                                int in, int padded, int dev, float scale, int kind,
                                                                int8_t *__restrict__ q, float *__restrict__ xs,
                                                                float *__restrict__ xst, int groups) {
    const int v = blockIdx.y;
    const int p = blockIdx.x * 256 + threadIdx.x;
    const int t = threadIdx.x & 63;
    const float *xv = (xptr ? xptr[v / batch] : x0) + static_cast<size_t>(v % batch) * in;
    const float r = p < in ? xv[p] : 0.0f;
    prepare_lane<GROUP>(r, t, p, padded, dev, scale, kind, q + static_cast<size_t>(v) * dev,
                        xs + static_cast<size_t>(v) * groups + p / GROUP,
                        xst ? xst + (static_cast<size_t>(v / batch) * groups + p / GROUP) * batch + v % batch : nullptr);
}

// Prepare for groups of 8 .. 64 positions with eight consecutive positions
// per thread (8 times fewer workgroups than sdot_prepare_wave_kernel, and
// 4-bit codes stored as one 8-byte word per thread): FWHT stages 1, 2, 4
// between the thread's own values, then stages 8 .. GROUP / 2 as in-wave
// butterflies on each value (the reference's stage order and operands), the
// group absmax over the thread's values and GROUP / 8 lanes, then the
// reference's quantiser as prepare_lane does it. Same values as
// sdot_prepare_kernel, bit for bit.
template <int GROUP>
__global__ __launch_bounds__(256) void sdot_prepare_oct_kernel(const float *__restrict__ x0,
                                                               const float *const *__restrict__ xptr, int batch,
                                                               int in, int padded, int dev, float scale, int kind,
                                                               int8_t *__restrict__ q, float *__restrict__ xs,
                                                               float *__restrict__ xst, int groups) {
    constexpr int L = GROUP / 8;  // lanes per group
    const int v = blockIdx.y;
    const int p0 = (blockIdx.x * 256 + static_cast<int>(threadIdx.x)) * 8;
    const int t = threadIdx.x & 63;
    const float *xv = (xptr ? xptr[v / batch] : x0) + static_cast<size_t>(v % batch) * in;
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(xv, static_cast<uint32_t>(in) * 4u);  // past `in`: zeros
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        r[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xr, static_cast<uint32_t>(p0 + i) * 4u, 0, 0));
#pragma unroll
    for (int h = 1; h < 8 && h < GROUP; h *= 2)  // stages 1, 2, 4 within the thread
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (!(i & h)) {
                const float a = r[i], b = r[i + h];
                r[i] = a + b;
                r[i + h] = a - b;
            }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        wave_butterflies<L, 1>(r[i], t);  // stages 8 .. GROUP / 2 (lane strides 1 .. L / 2)
        r[i] = r[i] * scale;
        m = fmaxf(m, fabsf(r[i]));
    }
    const float absmax = group_max<L>(m, t);
    float sc = absmax > 0 ? absmax / 127 : 1;  // sdot.cpp:77-81
    if (sc == 0.0f) sc = absmax;                // subnormal absmax/127 underflows
    uint32_t out[2] = {0u, 0u};                 // the 8 codes in the 4-bit permuted order
    int8_t qb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        int8_t c = 0;
        if (p0 + i < padded) {
            float val = rintf(r[i] / sc);
            val = val < -127.0f ? -127.0f : (127.0f < val ? 127.0f : val);
            c = static_cast<int8_t>(val);
        }
        qb[i] = c;
        out[i & 1] |= static_cast<uint32_t>(static_cast<uint8_t>(c)) << (8 * (i >> 1));
    }
    if (p0 >= dev) return;  // whole groups past the row (dev is a multiple of 256); no lane exchange follows
    int8_t *qv = q + static_cast<size_t>(v) * dev;
    if (kind == kNib) {
        *reinterpret_cast<uint2 *>(qv + p0) = make_uint2(out[0], out[1]);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) qv[permuted_index(kind, p0 + i)] = qb[i];
    }
    if (p0 % GROUP == 0 && p0 < padded) {
        xs[static_cast<size_t>(v) * groups + p0 / GROUP] = sc;
        if (xst) xst[(static_cast<size_t>(v / batch) * groups + p0 / GROUP) * batch + v % batch] = sc;
    }
}

// Prepare for groups of 128 and 256 positions, one wave per group without
// LDS (prepare_group_wave). Same values as sdot_prepare_kernel, bit for bit.
template <int GROUP>
__global__ __launch_bounds__(256) void sdot_prepare_wave_group_kernel(const float *__restrict__ x0,
                                                                      const float *const *__restrict__ xptr, int batch,
                                                                      int in, int padded, int dev, float scale,
                                                                      int kind, int8_t *__restrict__ q,
                                                                      float *__restrict__ xs, float *__restrict__ xst,
                                                                      int groups) {
    constexpr int VPL = GROUP / 64;  // values per lane
    const int v = blockIdx.y;
    const int t = threadIdx.x & 63;
    const int base = (blockIdx.x * 4 + static_cast<int>(threadIdx.x >> 6)) * GROUP;  // wave-uniform
    if (base >= dev) return;
    const float *xv = (xptr ? xptr[v / batch] : x0) + static_cast<size_t>(v % batch) * in;
    float r[VPL];
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
        const int p = base + t + 64 * k;
        r[k] = p < in ? xv[p] : 0.0f;
    }
    prepare_group_wave<GROUP>(r, t, base, padded, dev, scale, kind, q + static_cast<size_t>(v) * dev,
                              xs + static_cast<size_t>(v) * groups + base / GROUP,
                              xst ? xst + (static_cast<size_t>(v / batch) * groups + base / GROUP) * batch + v % batch
                                  : nullptr);
}

}  // namespace

// Groups of 8 .. 64 of at least 2^20 positions in all take the
// eight-positions-per-thread kernel (batch 16 of the 64 x 4096 stack:
// 17.8 -> ~12 us); a decode layer's 64 x 512 inputs keep one position per
// thread, whose latency is shorter (Q|K|V plan 7.6 -> 7.1 us).
// NEEDLE2_GPU_INT8_PREPARE = oct / lane overrides.
static bool prepare_oct_wanted(long values) {
    const char *mode = std::getenv("NEEDLE2_GPU_INT8_PREPARE");
    if (mode && std::strcmp(mode, "lane") == 0) return false;
    if (mode && std::strcmp(mode, "oct") == 0) return true;
    return values >= (1L << 20);
}

bool launch_sdot_prepare(const float *x0, const float *const *xptr, int batch, int nvec, int in, int padded,
                         int dev, int group, float scale, int kind, int32_t *q, float *xs, float *xst, hipStream_t s) {
    if (group > kPrepareMaxGroup) return false;
    ND_CHECK(group >= 8 && (group & (group - 1)) == 0, "int8 prepare: group must be a power of two >= 8");
    if (nvec <= 0) return true;
    if (group <= 64 && prepare_oct_wanted(static_cast<long>(nvec) * dev)) {
        dim3 grid((dev + 2047) / 2048, nvec), block(256);
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, block, 0, s, x0, xptr, batch, in, padded, dev, scale, kind,
                               reinterpret_cast<int8_t *>(q), xs, xst, padded / group);
        };
        switch (group) {
        case 8: go(sdot_prepare_oct_kernel<8>); break;
        case 16: go(sdot_prepare_oct_kernel<16>); break;
        case 32: go(sdot_prepare_oct_kernel<32>); break;
        default: go(sdot_prepare_oct_kernel<64>); break;
        }
        ND_HIP(hipGetLastError());
        return true;
    }
    if (group <= 64) {
        dim3 grid(dev / 256, nvec), block(256);
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, block, 0, s, x0, xptr, batch, in, padded, dev, scale, kind,
                               reinterpret_cast<int8_t *>(q), xs, xst, padded / group);
        };
        switch (group) {
        case 8: go(sdot_prepare_wave_kernel<8>); break;
        case 16: go(sdot_prepare_wave_kernel<16>); break;
        case 32: go(sdot_prepare_wave_kernel<32>); break;
        default: go(sdot_prepare_wave_kernel<64>); break;
        }
        ND_HIP(hipGetLastError());
        return true;
    }
    if (group <= 256) {
        dim3 grid((dev + 4 * group - 1) / (4 * group), nvec), block(256);
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, block, 0, s, x0, xptr, batch, in, padded, dev, scale, kind,
                               reinterpret_cast<int8_t *>(q), xs, xst, padded / group);
        };
        if (group == 128) go(sdot_prepare_wave_group_kernel<128>);
        else go(sdot_prepare_wave_group_kernel<256>);
        ND_HIP(hipGetLastError());
        return true;
    }
    const int seg = group > kPrepareMinSeg ? group : kPrepareMinSeg;
    dim3 grid((dev + seg - 1) / seg, nvec), block(256);
    hipLaunchKernelGGL(sdot_prepare_kernel, grid, block, seg * sizeof(float), s, x0, xptr, batch, in, padded, dev,
                       group, scale, kind, reinterpret_cast<int8_t *>(q), xs, xst, padded / group, seg);
    ND_HIP(hipGetLastError());
    return true;
}

void launch_sdot_quantize(const float *rot, int rot_stride, int nvec, int padded, int dev, int group, int kind,
                          int32_t *q, float *xs, hipStream_t s) {
    if (nvec <= 0) return;
    const int groups = padded / group;
    const int seg = group > 256 ? group : 256;
    dim3 grid((dev + seg - 1) / seg, nvec), block(256);
    hipLaunchKernelGGL(sdot_quantize_kernel, grid, block, 0, s, rot, rot_stride, padded, dev, group, kind,
                       reinterpret_cast<int8_t *>(q), xs, groups, seg);
    ND_HIP(hipGetLastError());
}

// 16-row batch tiles from 9 rows up (NEEDLE2_GPU_INT8_TILE16: "always" from
// 2 rows, "never"). At 8 rows the 4-row quads (two per weight row) measured
// 162-167 us per 64 x 4096^2 g32 stack against 172-173 us for half-filled
// 16-row tiles; at 12 rows three quads take 251 us, the tiles 178 us.
static bool tile16_wanted(int batch) {
    const char *mode = std::getenv("NEEDLE2_GPU_INT8_TILE16");
    if (mode && std::strcmp(mode, "never") == 0) return false;
    if (mode && std::strcmp(mode, "always") == 0) return batch >= 2;
    return batch > 8;
}

// The K split for small matrices (NEEDLE2_GPU_INT8_KSPLIT "always" / "never") and, within it, the 16 x 16
// tiles (batch 2 and more; NEEDLE2_GPU_INT8_KS16 "never", or "always" from batch 1).
static bool ks_chosen(const SdotGeom &g, int blocks, int batch) {
    const long mfma_waves = static_cast<long>(blocks) * (kRowsPerBlock / 32) * ((batch + 31) / 32);
    const char *ks_mode = std::getenv("NEEDLE2_GPU_INT8_KSPLIT");
    const bool ks_ok = g.group >= 32 && g.group <= kWindow && g.groups >= 2;
    bool ks = ks_ok && mfma_waves < 4L * device_cus();
    if (ks_mode && std::strcmp(ks_mode, "always") == 0) ks = ks_ok;
    if (ks_mode && std::strcmp(ks_mode, "never") == 0) ks = false;
    return ks;
}

static bool ks16_chosen(const SdotGeom &g, int batch) {
    const char *ks16_mode = std::getenv("NEEDLE2_GPU_INT8_KS16");
    return !(ks16_mode && std::strcmp(ks16_mode, "never") == 0) &&
           (batch >= 2 || (ks16_mode && std::strcmp(ks16_mode, "always") == 0));
}

// The XIN kernel's LDS: the prepared row and its scales beside the 16 KiB of parked terms.
constexpr size_t kXinMaxLds = 32 * 1024;

bool sdot_gemv_takes_x(const SdotGeom &g, int blocks, int batch) {
    const char *mode = std::getenv("NEEDLE2_GPU_INT8_XIN");
    if (mode && std::strcmp(mode, "never") == 0) return false;
    const size_t lds = static_cast<size_t>(g.windows) * kWindow + static_cast<size_t>(g.groups) * 4;
    return batch == 1 && g.group >= 32 && g.group <= kWindow && lds <= kXinMaxLds && ks_chosen(g, blocks, 1) &&
           !ks16_chosen(g, 1);
}

void launch_sdot_gemv_x(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks,
                        hipStream_t s) {
    ND_CHECK(sdot_gemv_takes_x(g, blocks, 1), "internal: int8 GEMV with in-kernel prepare outside its shapes");
    if (g.kind == kNib) launch_sdot_ks_j<kNib, 1, true>(g, job0, jobs, njobs, blocks, 1, s);
    else launch_sdot_ks_j<kCrumb, 1, true>(g, job0, jobs, njobs, blocks, 1, s);
}

bool launch_sdot_gemv_prep(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks,
                           int batch, const PrepOut &po, hipStream_t s) {
    if (blocks <= 0 || batch <= 0 || !po.q || g.group < 32 || g.group > kWindow) return false;
    if (!ks_chosen(g, blocks, batch) || !ks16_chosen(g, batch)) return false;
    if (g.kind == kNib) launch_sdot_ks16_kind<kNib, 2, true>(g, job0, jobs, njobs, blocks, batch, po, s);
    else launch_sdot_ks16_kind<kCrumb, 2, true>(g, job0, jobs, njobs, blocks, batch, po, s);
    return true;
}

void launch_sdot_gemv(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks, int batch,
                      hipStream_t s) {
    if (blocks <= 0 || batch <= 0) return;
    ND_CHECK(g.group >= 8, "int8 path: group must be >= 8");
    ND_CHECK(g.kind == kNib || g.group >= 16, "int8 path: 2-bit codes need group >= 16");
    // Kernel by size (environment overrides, "always" / "never", let the
    // tests run every kernel on every shape):
    //  - small matrices (fewer 32 x 32 tiles than SIMDs: decode projections)
    //    of any batch split K over 8 or 16 waves per tile (NEEDLE2_GPU_INT8_KSPLIT),
    //    on 16 x 16 tiles at batch 2 and more (NEEDLE2_GPU_INT8_KS16:
    //    "never", or "always" from batch 1);
    //  - one batch row: the barrier-free row kernel (NEEDLE2_GPU_INT8_ROW);
    //  - 9 or more: batch tiles of 16 rows on v_mfma_i32_16x16x32_i8, every
    //    code decoded once per tile (NEEDLE2_GPU_INT8_TILE16);
    //  - 2 or more: batch tiles of up to 16 rows on v_mfma_i32_4x4x4_16b_i8,
    //    one lane per weight row, every code decoded once per tile
    //    (NEEDLE2_GPU_INT8_QUAD);
    //  - otherwise 32 x 32 batch tiles on v_mfma_i32_32x32x32_i8 for 8 or
    //    more rows (NEEDLE2_GPU_INT8_MFMA) and v_dot4 batch tiles below.
    const long mfma_waves = static_cast<long>(blocks) * (kRowsPerBlock / 32) * ((batch + 31) / 32);
    const char *mode = std::getenv("NEEDLE2_GPU_INT8_MFMA");
    const char *quad_mode = std::getenv("NEEDLE2_GPU_INT8_QUAD");
    if (ks_chosen(g, blocks, batch)) {
        if (ks16_chosen(g, batch) && launch_sdot_ks16(g, job0, jobs, njobs, blocks, batch, s)) return;
        if (g.kind == kNib) launch_sdot_ks<kNib>(g, job0, jobs, njobs, blocks, batch, s);
        else launch_sdot_ks<kCrumb>(g, job0, jobs, njobs, blocks, batch, s);
        return;
    }
    const bool mfma_ok = batch >= 2 && g.group >= 32 && g.group <= kWindow;
    const bool mfma_forced = mode && std::strcmp(mode, "always") == 0;
    const char *row_mode = std::getenv("NEEDLE2_GPU_INT8_ROW");
    if (!mfma_forced && batch == 1 && g.group <= kWindow && g.windows * kWindow <= kRowMaxDev &&
        !(row_mode && std::strcmp(row_mode, "never") == 0)) {
        if (g.kind == kNib) launch_sdot_row<kNib, false>(g, job0, jobs, njobs, blocks, nullptr, s);
        else launch_sdot_row<kCrumb, false>(g, job0, jobs, njobs, blocks, nullptr, s);
        return;
    }
    if (!mfma_forced && tile16_wanted(batch)) {
        const bool done = g.kind == kNib ? launch_sdot_tile16<kNib, false>(g, job0, jobs, njobs, blocks, batch, nullptr, s)
                                         : launch_sdot_tile16<kCrumb, false>(g, job0, jobs, njobs, blocks, batch, nullptr, s);
        if (done) return;
    }
    if (!mfma_forced && batch >= 2 && !(quad_mode && std::strcmp(quad_mode, "never") == 0)) {
        const bool done = g.kind == kNib ? launch_sdot_quad<kNib, false>(g, job0, jobs, njobs, blocks, batch, nullptr, s)
                                         : launch_sdot_quad<kCrumb, false>(g, job0, jobs, njobs, blocks, batch, nullptr, s);
        if (done) return;
    }
    bool mfma = mfma_ok && batch >= 8 && mfma_waves >= 2L * 4 * device_cus();
    if (mfma_forced) mfma = mfma_ok;
    if (mode && std::strcmp(mode, "never") == 0) mfma = false;
    if (mfma) {
        if (g.kind == kNib) launch_sdot_mfma<kNib>(g, job0, jobs, njobs, blocks, batch, s);
        else launch_sdot_mfma<kCrumb>(g, job0, jobs, njobs, blocks, batch, s);
        return;
    }
    if (g.kind == kNib) launch_sdot_kind<kNib>(g, job0, jobs, njobs, blocks, batch, s);
    else launch_sdot_kind<kCrumb>(g, job0, jobs, njobs, blocks, batch, s);
}

void launch_sdot_dots(const SdotGeom &g, const SdotJob &job0, int blocks, int batch, int32_t *dots, hipStream_t s) {
    if (blocks <= 0 || batch <= 0) return;
    ND_CHECK(g.group >= 8 && g.group <= kWindow, "int8 dots: groups of 8 .. 256");
    ND_CHECK(g.kind == kNib || g.group >= 16, "int8 path: 2-bit codes need group >= 16");
    if (batch == 1) {
        ND_CHECK(g.windows * kWindow <= kRowMaxDev, "int8 dots: the row exceeds the batch-1 kernel's stage");
        if (g.kind == kNib) launch_sdot_row<kNib, true>(g, job0, nullptr, 0, blocks, dots, s);
        else launch_sdot_row<kCrumb, true>(g, job0, nullptr, 0, blocks, dots, s);
        return;
    }
    bool done = false;
    if (tile16_wanted(batch))
        done = g.kind == kNib ? launch_sdot_tile16<kNib, true>(g, job0, nullptr, 0, blocks, batch, dots, s)
                              : launch_sdot_tile16<kCrumb, true>(g, job0, nullptr, 0, blocks, batch, dots, s);
    if (!done)
        done = g.kind == kNib ? launch_sdot_quad<kNib, true>(g, job0, nullptr, 0, blocks, batch, dots, s)
                              : launch_sdot_quad<kCrumb, true>(g, job0, nullptr, 0, blocks, batch, dots, s);
    ND_CHECK(done, "int8 dots: the batch tile exceeds the kernel's LDS stage");
}

}  // namespace nd
