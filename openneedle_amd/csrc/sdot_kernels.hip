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
// against activations held in scalar registers (uniform across the wave).
// The int32 group dot is exact in any order; the epilogue is the reference's
//   value += (float(dot) * (half(norm) * cs)) * x_scale[g]
// sequentially over g (sdot.cpp:43-44, 142-149), so outputs are bit-exact.
#include "common.h"

#include <hip/hip_fp16.h>

namespace nd {

namespace {

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// position p within a row -> byte index in the permuted int8 activation row
__device__ __forceinline__ int permuted_index(int kind, int p) {
    if (kind == kNib) {
        int d = p >> 3, i = p & 7;  // codes 0,2,4,6 then 1,3,5,7 of each 8-code dword
        return (d << 3) | ((i & 1) << 2) | (i >> 1);
    }
    int d = p >> 4, i = p & 15;  // selector m = i&3 holds crumbs m, m+4, m+8, m+12
    return (d << 4) | ((i & 3) << 2) | (i >> 2);
}

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

// ---------------------------------------------------------------------------
// GEMV
// ---------------------------------------------------------------------------
// 8 four-bit codes (one dword) -> int8 centroids for codes {0,2,4,6} and {1,3,5,7}.
__device__ __forceinline__ void decode_nib(uint32_t w, uint32_t T0, uint32_t T1, uint32_t T2, uint32_t T3,
                                           uint32_t &ce, uint32_t &co) {
    const uint32_t e = w & 0x07070707u, o = (w >> 4) & 0x07070707u;
    const uint32_t le = __builtin_amdgcn_perm(T1, T0, e), he = __builtin_amdgcn_perm(T3, T2, e);
    const uint32_t lo = __builtin_amdgcn_perm(T1, T0, o), ho = __builtin_amdgcn_perm(T3, T2, o);
    const uint32_t se = ((w >> 1) & 0x04040404u) | 0x03020100u;  // bit 3 of each code picks high half
    const uint32_t so = ((w >> 5) & 0x04040404u) | 0x03020100u;
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

template <int KIND, int GROUP>
__device__ __forceinline__ void sdot_load(SdotWindow<KIND, GROUP> &st, const ND_GLOBAL u32x4 *__restrict__ codes,
                                          const ND_GLOBAL uint16_t *__restrict__ norms, int n_pad, int row, int w,
                                          int groups, int wpg) {
    constexpr int C = SdotWindow<KIND, GROUP>::kChunks;
    constexpr int NN = SdotWindow<KIND, GROUP>::kNorms;
    const ND_GLOBAL u32x4 *cw = codes + static_cast<size_t>(w) * C * n_pad + row;
#pragma unroll
    for (int c = 0; c < C; ++c) st.codes[c] = cw[static_cast<size_t>(c) * n_pad];
    // clamped group indices: unconditional loads (phantom groups are never closed)
    if constexpr (GROUP > 0) {
#pragma unroll
        for (int k = 0; k < NN; ++k) {
            const int g = min(w * NN + k, groups - 1);
            st.norms[k] = norms[static_cast<size_t>(g) * n_pad + row];
        }
    } else {
        const int g = min(w / wpg, groups - 1);
        st.norms[0] = norms[static_cast<size_t>(g) * n_pad + row];
    }
}

template <int KIND, int GROUP>
__device__ __forceinline__ void sdot_compute(const SdotWindow<KIND, GROUP> &st, const ND_CONST int32_t *__restrict__ qw,
                                             const ND_CONST float *__restrict__ xs, const uint32_t cent[4], float cs,
                                             float &value, int &dot, int w, int groups, int wpg) {
    constexpr int C = SdotWindow<KIND, GROUP>::kChunks;
    constexpr int NN = SdotWindow<KIND, GROUP>::kNorms;
    const int gbase = w * NN;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const uint32_t words[4] = {st.codes[c].x, st.codes[c].y, st.codes[c].z, st.codes[c].w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t wd = words[d];
            if constexpr (KIND == kNib) {
                uint32_t ce, co;
                decode_nib(wd, cent[0], cent[1], cent[2], cent[3], ce, co);
                const int qi = (c * 4 + d) * 2;
                dot = __builtin_amdgcn_sdot4(static_cast<int>(ce), qw[qi], dot, false);
                dot = __builtin_amdgcn_sdot4(static_cast<int>(co), qw[qi + 1], dot, false);
                if constexpr (GROUP > 0) {
                    const int pos_end = (c * 4 + d + 1) * 8;
                    if (pos_end % GROUP == 0) {
                        const int k = pos_end / GROUP - 1;
                        if (gbase + k < groups)
                            value += (static_cast<float>(dot) * (h2f(st.norms[k]) * cs)) * xs[gbase + k];
                        dot = 0;
                    }
                }
            } else {
                const int qi = (c * 4 + d) * 4;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const uint32_t sel = (wd >> (2 * m)) & 0x03030303u;
                    const uint32_t cc = __builtin_amdgcn_perm(0u, cent[0], sel);
                    dot = __builtin_amdgcn_sdot4(static_cast<int>(cc), qw[qi + m], dot, false);
                }
                if constexpr (GROUP > 0) {
                    const int pos_end = (c * 4 + d + 1) * 16;
                    if (pos_end % GROUP == 0) {
                        const int k = pos_end / GROUP - 1;
                        if (gbase + k < groups)
                            value += (static_cast<float>(dot) * (h2f(st.norms[k]) * cs)) * xs[gbase + k];
                        dot = 0;
                    }
                }
            }
        }
    }
    if constexpr (GROUP == 0) {
        if ((w + 1) % wpg == 0) {
            const int g = w / wpg;
            if (g < groups) value += (static_cast<float>(dot) * (h2f(st.norms[0]) * cs)) * xs[g];
            dot = 0;
        }
    }
}

template <int KIND, int GROUP>
__global__ __launch_bounds__(kRowsPerBlock) void sdot_gemv_kernel(SdotJob job0, const SdotJob *__restrict__ jobs,
                                                                  int njobs, SdotGeom geom) {
    const int blk = blockIdx.x;
    SdotJob J = job0;
    if (njobs > 0) {
        const ND_CONST SdotJob *cj = (const ND_CONST SdotJob *)(jobs);
        int j = 0;
        for (int k = 1; k < njobs; ++k)
            if (cj[k].block_begin <= blk) j = k;
        J.codes = cj[j].codes;
        J.norms = cj[j].norms;
        J.q = cj[j].q;
        J.xs = cj[j].xs;
        J.y = cj[j].y;
        J.rows = cj[j].rows;
        J.n_pad = cj[j].n_pad;
        J.block_begin = cj[j].block_begin;
        J.batch = cj[j].batch;
    }
    const ND_GLOBAL u32x4 *__restrict__ codes = (const ND_GLOBAL u32x4 *)(J.codes);
    const ND_GLOBAL uint16_t *__restrict__ norms = (const ND_GLOBAL uint16_t *)(J.norms);
    const int n_pad = J.n_pad, rows = J.rows, batch = J.batch;
    const int row = (blk - J.block_begin) * kRowsPerBlock + threadIdx.x;
    const int windows = geom.windows, groups = geom.groups;
    const int wpg = GROUP == 0 ? geom.group / kWindow : 1;
    const int qdw = windows * (kWindow / 4);  // int32 activation words per batch row
    const uint32_t cent[4] = {geom.cent[0], geom.cent[1], geom.cent[2], geom.cent[3]};
    const float cs = geom.centroid_scale;

    for (int b = 0; b < batch; ++b) {
        const ND_CONST int32_t *__restrict__ q = (const ND_CONST int32_t *)(J.q) + static_cast<size_t>(b) * qdw;
        const ND_CONST float *__restrict__ xs = (const ND_CONST float *)(J.xs) + static_cast<size_t>(b) * groups;
        SdotWindow<KIND, GROUP> cur, nxt;
        sdot_load<KIND, GROUP>(cur, codes, norms, n_pad, row, 0, groups, wpg);
        float value = 0.0f;
        int dot = 0;
        for (int w = 0; w < windows; w += 2) {
            if (w + 1 < windows) sdot_load<KIND, GROUP>(nxt, codes, norms, n_pad, row, w + 1, groups, wpg);
            sdot_compute<KIND, GROUP>(cur, q + w * (kWindow / 4), xs, cent, cs, value, dot, w, groups, wpg);
            if (w + 1 >= windows) break;
            if (w + 2 < windows) sdot_load<KIND, GROUP>(cur, codes, norms, n_pad, row, w + 2, groups, wpg);
            sdot_compute<KIND, GROUP>(nxt, q + (w + 1) * (kWindow / 4), xs, cent, cs, value, dot, w + 1, groups, wpg);
        }
        if (row < rows) ((ND_GLOBAL float *)J.y)[static_cast<size_t>(b) * rows + row] = value;
    }
}

template <int KIND>
void launch_sdot_kind(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks,
                      hipStream_t s) {
    dim3 grid(blocks), block(kRowsPerBlock);
    switch (g.group > kWindow ? 0 : g.group) {
    case 16: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 16>), grid, block, 0, s, job0, jobs, njobs, g); break;
    case 32: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 32>), grid, block, 0, s, job0, jobs, njobs, g); break;
    case 64: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 64>), grid, block, 0, s, job0, jobs, njobs, g); break;
    case 128: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 128>), grid, block, 0, s, job0, jobs, njobs, g); break;
    case 256: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 256>), grid, block, 0, s, job0, jobs, njobs, g); break;
    default: hipLaunchKernelGGL((sdot_gemv_kernel<KIND, 0>), grid, block, 0, s, job0, jobs, njobs, g); break;
    }
    ND_HIP(hipGetLastError());
}

}  // namespace

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

void launch_sdot_gemv(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs, int njobs, int blocks,
                      hipStream_t s) {
    if (blocks <= 0) return;
    ND_CHECK(g.group >= 8, "int8 path: group must be >= 8");
    ND_CHECK(g.kind == kNib || g.group >= 16, "int8 path: 2-bit codes need group >= 16");
    if (g.kind == kNib) {
        if (g.group == 8) {
            dim3 grid(blocks), block(kRowsPerBlock);
            hipLaunchKernelGGL((sdot_gemv_kernel<kNib, 8>), grid, block, 0, s, job0, jobs, njobs, g);
            ND_HIP(hipGetLastError());
        } else {
            launch_sdot_kind<kNib>(g, job0, jobs, njobs, blocks, s);
        }
    } else {
        launch_sdot_kind<kCrumb>(g, job0, jobs, njobs, blocks, s);
    }
}

}  // namespace nd
