// gfx950 prefill GEMM: Y[m][n] = sum_k FWHT(X)[m][k] * cb[code[n][k]] * norm[n][k / group]
// on fp16 MFMA with fp32 accumulation (the batched form of cq.cpp:157-197,
// as Engine::linear_batch uses it for prompt chunks, engine.cpp:607-670).
//
// 1. prefill_transform_kernel: per-group FWHT of X (the reference's stage
//    order, then * 1/sqrt(group)) written as fp16 in MFMA fragment order:
//    each 16-byte slice is one lane's operand of one v_mfma_f32_32x32x16_f16,
//    so the GEMM loads X fragments straight from memory (1 KiB per wave load).
// 2. prefill_gemm_kernel: 128 x 128 output tile per workgroup, K in steps of
//    64 positions, two kinds of waves. Waves 0-3 (one per SIMD) each own a
//    64 x 64 sub-tile: X fragments from memory two steps ahead, weight
//    fragments from LDS, 16 MFMAs per step. Waves 4-7 (one per SIMD) load
//    the 4-bit codes three steps ahead and dequantize the 128 x 64 weight
//    tile of the next step into the other LDS buffer: codes -> fp16 codebook
//    values through v_perm byte tables, times the fp16 group norm. One
//    barrier per step; on each SIMD the dequantization VALU work issues while
//    the MFMA wave's matrix instructions run. Tiles are ordered so that the
//    M-tiles of one N-tile run on the same XCD and share its L2.
//
// Rounding: X and the weights cb*norm are fp16 (two roundings for the
// weight), products and sums are fp32 in the MFMA; the result agrees with the
// reference FP32 path to about 1e-3 normwise (bound 2e-3).
#include "common.h"

#include <hip/hip_fp16.h>

namespace nd {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));

namespace {

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kGemmThreads = 512;  // waves 0-3: MFMA (2 x 2 of 64 x 64); waves 4-7: weight dequantization
constexpr int kLdsRow = 72;        // halves per LDS weight row: 64 + 8 padding (conflict-free 16-byte accesses)
constexpr int kFragBytes = 1024;   // one operand fragment: 64 lanes x 8 halves
constexpr int kStepBytes = 4 * kFragBytes;  // the four 16-position slices of one 64-position step

// Half e (0..7) of a lane's 8-half slice holds position 8 d + kCidx(e) of its
// code dword d: the order dequant8 produces (0,2,4,6,1,3,5,7).
__host__ __device__ constexpr int cidx(int e) { return (e & 3) * 2 + (e >> 2); }

// FWHT as transform_kernel, fp16 output in fragment order: for 32-row block
// rb, step s and slice kk, lane l holds row 32 rb + l % 32 and positions
// 64 s + 32 (l / 32) + 8 kk + cidx(e). Rows m .. m32 - 1 are written as zeros.
__global__ __launch_bounds__(256) void prefill_transform_kernel(const float *__restrict__ x, int m, int in, int padded,
                                                                int dev, int group, float scale,
                                                                _Float16 *__restrict__ xf, int seg) {
    extern __shared__ float buf[];
    const int v = blockIdx.y;
    const int base = blockIdx.x * seg;
    const bool live = v < m;
    const float *xv = x + static_cast<size_t>(live ? v : 0) * in;
    for (int i = threadIdx.x; i < seg; i += blockDim.x) {
        const int p = base + i;
        buf[i] = live && p < in ? xv[p] : 0.0f;
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
    const size_t block = static_cast<size_t>(v >> 5) * (dev / kBK);
    for (int u = threadIdx.x; u < seg / 8; u += blockDim.x) {
        const int p0 = base + 8 * u;
        if (p0 >= dev) break;
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int c0 = cidx(2 * q), c1 = cidx(2 * q + 1);
            const _Float16 h0 = static_cast<_Float16>(p0 + c0 < padded ? buf[8 * u + c0] * scale : 0.0f);
            const _Float16 h1 = static_cast<_Float16>(p0 + c1 < padded ? buf[8 * u + c1] * scale : 0.0f);
            w[q] = uint32_t(__builtin_bit_cast(uint16_t, h0)) | (uint32_t(__builtin_bit_cast(uint16_t, h1)) << 16);
        }
        const int s = p0 >> 6, hh = (p0 >> 5) & 1, kk = (p0 >> 3) & 3;
        const size_t idx = (((block + s) * 4 + kk) * 64 + hh * 32 + (v & 31)) * 8;
        *reinterpret_cast<u32x4 *>(xf + idx) = u32x4{w[0], w[1], w[2], w[3]};
    }
}

// Byte lookups in a 16-entry table T (4 dwords) for the 4 byte-wide indices
// of a code vector: i7 = idx & 7 per byte, sel picks the upper 8 entries.
struct LutIdx {
    uint32_t i7, sel;
};
__device__ __forceinline__ LutIdx lut_idx(uint32_t idx) {
    return {idx & 0x07070707u, ((idx >> 1) & 0x04040404u) | 0x03020100u};
}
__device__ __forceinline__ uint32_t lut16(LutIdx x, const uint32_t (&T)[4]) {
    const uint32_t lo = __builtin_amdgcn_perm(T[1], T[0], x.i7), hi = __builtin_amdgcn_perm(T[3], T[2], x.i7);
    return __builtin_amdgcn_perm(hi, lo, x.sel);
}

// 8 four-bit codes (LSB first) -> 8 fp16 codebook values times the fp16 norm
// (both halves of `norm2`), in the order 0,2,4,6,1,3,5,7 (the activations are
// stored in the same order), which saves re-interleaving.
__device__ __forceinline__ void dequant8(uint32_t w, const uint32_t (&LO)[4], const uint32_t (&HI)[4], uint32_t norm2,
                                         uint32_t (&out)[4]) {
    const LutIdx e = lut_idx(w & 0x0F0F0F0Fu), o = lut_idx((w >> 4) & 0x0F0F0F0Fu);  // codes 0,2,4,6 / 1,3,5,7
    const uint32_t le = lut16(e, LO), he = lut16(e, HI), lo = lut16(o, LO), ho = lut16(o, HI);
    const uint32_t v[4] = {__builtin_amdgcn_perm(he, le, 0x05010400u),   // codes 0 | 2
                           __builtin_amdgcn_perm(he, le, 0x07030602u),   // 4 | 6
                           __builtin_amdgcn_perm(ho, lo, 0x05010400u),   // 1 | 3
                           __builtin_amdgcn_perm(ho, lo, 0x07030602u)};  // 5 | 7
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 n = __builtin_bit_cast(h2, norm2);
#pragma unroll
    for (int q = 0; q < 4; ++q) out[q] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v[q]) * n);
}

struct GemmArgs {
    const _Float16 *xf;  // X in fragment order (prefill_transform_kernel), rb_count blocks of 32 rows
    const uint4 *codes;  // matrix device layout (4-bit codes)
    const uint16_t *norms;
    float *y;  // [m][rows]
    int m, rb_count, rows, chunks, groups, group_shift, xsteps, ksteps, mtiles, tiles;
    uint32_t lo[4], hi[4];  // fp16 codebook, low / high byte tables
};

// Tile of this workgroup. Workgroups go to the 8 XCDs round robin; giving
// each XCD a contiguous run of tiles (M-tile fastest) keeps the M-tiles of an
// N-tile, which read the same codes, on one XCD's L2.
__device__ __forceinline__ int gemm_tile(const GemmArgs &g) {
    const int b = blockIdx.x;
    return g.tiles % 8 ? b : (b & 7) * (g.tiles >> 3) + (b >> 3);
}

// ---- MFMA waves ----------------------------------------------------------

struct AFrags {
    u32x4 v[2][4];  // [32-row block i][slice kk]
};

struct APtrs {
    __amdgpu_buffer_rsrc_t x;
    uint32_t xv[2];  // lane offsets of the wave's two row blocks
};

__device__ __forceinline__ APtrs a_ptrs(const GemmArgs &g, int rb0, int lane) {
    const uint32_t block = static_cast<uint32_t>(g.xsteps) * kStepBytes;
    // blocks past the last read zero (scalar: a VALU clamp would make the descriptor divergent)
    const int left = __builtin_amdgcn_readfirstlane(min(2, max(0, g.rb_count - rb0)));
    APtrs p;
    p.x = buffer_rsrc(g.xf + static_cast<size_t>(rb0) * g.xsteps * (kStepBytes / 2), left * block);
    p.xv[0] = lane * 16u;
    p.xv[1] = lane * 16u + block;
    return p;
}

__device__ __forceinline__ void a_load(AFrags &a, const APtrs &p, int s) {
    const int so = __builtin_amdgcn_readfirstlane(s * kStepBytes);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            a.v[i][kk] = __builtin_amdgcn_raw_buffer_load_b128(p.x, p.xv[i] + kk * kFragBytes, so, 0);
}

struct BFrags {
    h8 v[4][2];  // [slice kk][32-column block j]
};

// Weight fragments of one step from LDS buffer `Bs`: lane l holds weight row
// l % 32 of the block, slice kk of chunk l / 32.
__device__ __forceinline__ void b_read(BFrags &b, const _Float16 *Bs, int wn, int lane) {
    const _Float16 *B = Bs + (wn * 64 + (lane & 31)) * kLdsRow + (lane >> 5) * 32;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int j = 0; j < 2; ++j) b.v[kk][j] = *reinterpret_cast<const h8 *>(B + j * 32 * kLdsRow + kk * 8);
}

// One K step of an MFMA wave (J = c % 6): X fragments of step c + 2 are
// requested (ring of three register sets), the weight fragments of step
// c + 1 are read from LDS buffer (c + 1) % 3 (complete since the previous
// barrier), and step c is computed from registers only.
template <int J>
__device__ __forceinline__ void mma_step(AFrags (&a)[3], BFrags (&b)[2], const GemmArgs &g, const APtrs &p, int c,
                                         const _Float16 (&Bs)[3][kBN * kLdsRow], f16x (&acc)[2][2], int wn,
                                         int lane) {
    a_load(a[(J + 2) % 3], p, min(c + 2, g.ksteps - 1));  // clamped: past the end it repeats the last step
    b_read(b[(J + 1) & 1], Bs[(J + 1) % 3], wn, lane);    // past the end: never used
    const AFrags &x = a[J % 3];
    const BFrags &w = b[J & 1];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, x.v[i][kk]), w.v[kk][j],
                                                                   acc[i][j], 0, 0, 0);
    __syncthreads();
}

// ---- dequantization waves ------------------------------------------------

// Codes of one step for one (weight row, 32-position chunk): 4 code dwords
// and the NG fp16 norms they use (NG = 4, 2, 1 for groups 8, 16, >= 32).
template <int NG>
struct CodeRegs {
    u32x4 code;
    uint32_t norm[NG];
};

struct DPtrs {
    __amdgpu_buffer_rsrc_t c, n;
    uint32_t cv, nv[4];
};

template <int NG>
__device__ __forceinline__ DPtrs d_ptrs(const GemmArgs &g, int n0, int row, int ch) {
    const int tile = n0 / kRowsPerBlock, r = n0 % kRowsPerBlock + row;  // row inside its 256-row tile
    DPtrs p;
    p.c = buffer_rsrc(g.codes + static_cast<size_t>(tile) * g.chunks * kRowsPerBlock,
                      static_cast<uint32_t>(g.chunks) * kRowsPerBlock * 16u);
    p.cv = (static_cast<uint32_t>(ch) * kRowsPerBlock + r) * 16u;
    // groups past the last (positions past `padded`) read zero through the bound
    p.n = buffer_rsrc(g.norms + static_cast<size_t>(tile) * g.groups * kRowsPerBlock,
                      static_cast<uint32_t>(g.groups) * kRowsPerBlock * 2u);
#pragma unroll
    for (int k = 0; k < NG; ++k) {
        const int q = 32 * ch + k * (32 / NG);  // first position of norm k inside the step
        const int gq = g.group_shift <= 6 ? q >> g.group_shift : 0;
        p.nv[k] = (static_cast<uint32_t>(gq) * kRowsPerBlock + r) * 2u;
    }
    return p;
}

template <int NG>
__device__ __forceinline__ void code_load(CodeRegs<NG> &r, const GemmArgs &g, const DPtrs &p, int s) {
    r.code = __builtin_amdgcn_raw_buffer_load_b128(p.c, p.cv, __builtin_amdgcn_readfirstlane(s * 2 * kRowsPerBlock * 16),
                                                   0);
    const int gs = g.group_shift <= 6 ? s << (6 - g.group_shift) : (s << 6) >> g.group_shift;  // step's first group
    const int so = __builtin_amdgcn_readfirstlane(gs * kRowsPerBlock * 2);
#pragma unroll
    for (int k = 0; k < NG; ++k) r.norm[k] = __builtin_amdgcn_raw_buffer_load_b16(p.n, p.nv[k], so, 0);
}

// Weight row `row`, chunk `ch` of one step -> LDS slots 32 ch .. + 32 of the row.
template <int NG>
__device__ __forceinline__ void dequant_store(const CodeRegs<NG> &r, const GemmArgs &g, _Float16 *Bs, int row,
                                              int ch) {
    const uint32_t c[4] = {r.code.x, r.code.y, r.code.z, r.code.w};
    u32x4 *d = reinterpret_cast<u32x4 *>(Bs + row * kLdsRow + ch * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t nm = r.norm[q * NG / 4];
        uint32_t w[4];
        dequant8(c[q], g.lo, g.hi, nm | (nm << 16), w);
        d[q] = u32x4{w[0], w[1], w[2], w[3]};
    }
}

// One K step of a dequantization wave (J = c % 6): codes of step c + 5 are
// requested (ring of six), step c + 2 is dequantized into LDS buffer
// (c + 2) % 3, which the MFMA waves last read during step c - 2.
template <int NG, int J>
__device__ __forceinline__ void deq_step(CodeRegs<NG> (&r)[6], const GemmArgs &g, const DPtrs &p, int c,
                                         _Float16 (&Bs)[3][kBN * kLdsRow], int row, int ch) {
    code_load(r[(J + 5) % 6], g, p, min(c + 5, g.ksteps - 1));
    if (c + 2 < g.ksteps) dequant_store(r[(J + 2) % 6], g, Bs[(J + 2) % 3], row, ch);
    __syncthreads();
}

template <int NG>
__global__ __launch_bounds__(kGemmThreads) void prefill_gemm_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) _Float16 Bs[3][kBN * kLdsRow];
    const int tile = gemm_tile(g);
    const int n0 = (tile / g.mtiles) * kBN, m0 = (tile % g.mtiles) * kBM;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int last = g.ksteps - 1;
    // Every step ends in one barrier on both sides; the loops run in sixes so
    // that every ring index is a compile-time constant.
    if (wave < 4) {
        const int wm = wave >> 1, wn = wave & 1;  // this wave: rows 64 wm.., columns 64 wn..
        const APtrs p = a_ptrs(g, m0 / 32 + 2 * wm, lane);
        f16x acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = f16x{};
        AFrags a[3];
        BFrags b[2];
        a_load(a[0], p, 0);
        a_load(a[1], p, min(1, last));
        __syncthreads();  // weights of steps 0 and 1 are in LDS
        b_read(b[0], Bs[0], wn, lane);
        int c = 0;
        for (; c + 6 <= g.ksteps; c += 6) {
            mma_step<0>(a, b, g, p, c, Bs, acc, wn, lane);
            mma_step<1>(a, b, g, p, c + 1, Bs, acc, wn, lane);
            mma_step<2>(a, b, g, p, c + 2, Bs, acc, wn, lane);
            mma_step<3>(a, b, g, p, c + 3, Bs, acc, wn, lane);
            mma_step<4>(a, b, g, p, c + 4, Bs, acc, wn, lane);
            mma_step<5>(a, b, g, p, c + 5, Bs, acc, wn, lane);
        }
        if (c < g.ksteps) mma_step<0>(a, b, g, p, c, Bs, acc, wn, lane);
        if (c + 1 < g.ksteps) mma_step<1>(a, b, g, p, c + 1, Bs, acc, wn, lane);
        if (c + 2 < g.ksteps) mma_step<2>(a, b, g, p, c + 2, Bs, acc, wn, lane);
        if (c + 3 < g.ksteps) mma_step<3>(a, b, g, p, c + 3, Bs, acc, wn, lane);
        if (c + 4 < g.ksteps) mma_step<4>(a, b, g, p, c + 4, Bs, acc, wn, lane);
        // C fragment: lane l holds column l % 32, rows 8 (e / 4) + 4 (l / 32) + e % 4
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= g.rows) continue;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int m = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                    if (m < g.m) g.y[static_cast<size_t>(m) * g.rows + n] = acc[i][j][e];
                }
        }
    } else {
        const int u = threadIdx.x - 256;
        const int row = u & (kBN - 1), ch = u >> 7;  // weight row of the tile, chunk of the step
        const DPtrs p = d_ptrs<NG>(g, n0, row, ch);
        CodeRegs<NG> r[6];
#pragma unroll
        for (int k = 0; k < 5; ++k) code_load(r[k], g, p, min(k, last));
        dequant_store(r[0], g, Bs[0], row, ch);
        if (1 < g.ksteps) dequant_store(r[1], g, Bs[1], row, ch);
        __syncthreads();
        int c = 0;
        for (; c + 6 <= g.ksteps; c += 6) {
            deq_step<NG, 0>(r, g, p, c, Bs, row, ch);
            deq_step<NG, 1>(r, g, p, c + 1, Bs, row, ch);
            deq_step<NG, 2>(r, g, p, c + 2, Bs, row, ch);
            deq_step<NG, 3>(r, g, p, c + 3, Bs, row, ch);
            deq_step<NG, 4>(r, g, p, c + 4, Bs, row, ch);
            deq_step<NG, 5>(r, g, p, c + 5, Bs, row, ch);
        }
        if (c < g.ksteps) deq_step<NG, 0>(r, g, p, c, Bs, row, ch);
        if (c + 1 < g.ksteps) deq_step<NG, 1>(r, g, p, c + 1, Bs, row, ch);
        if (c + 2 < g.ksteps) deq_step<NG, 2>(r, g, p, c + 2, Bs, row, ch);
        if (c + 3 < g.ksteps) deq_step<NG, 3>(r, g, p, c + 3, Bs, row, ch);
        if (c + 4 < g.ksteps) deq_step<NG, 4>(r, g, p, c + 4, Bs, row, ch);
    }
}

}  // namespace

size_t prefill_xf_halves(int m, int dev) { return static_cast<size_t>((m + 31) / 32) * 32 * dev; }

void launch_prefill_transform(const float *x, int m, int in, int padded, int dev, int group, float scale,
                              _Float16 *xf, hipStream_t s) {
    if (m <= 0) return;
    ND_CHECK(group <= 16384, "prefill GEMM: group must be <= 16384");
    ND_CHECK(dev % kBK == 0, "internal: prefill rows must be whole 64-position steps");
    const int seg = group > 1024 ? group : 1024;
    dim3 grid((dev + seg - 1) / seg, (m + 31) / 32 * 32), block(256);
    hipLaunchKernelGGL(prefill_transform_kernel, grid, block, seg * sizeof(float), s, x, m, in, padded, dev, group,
                       scale, xf, seg);
    ND_HIP(hipGetLastError());
}

void launch_prefill_gemm(const CqGeom &geom, const uint4 *codes, const uint16_t *norms, int rows, const _Float16 *xf,
                         int m, int dev, int padded, const uint16_t *cb_half, float *y, hipStream_t s) {
    if (m <= 0) return;
    ND_CHECK(geom.kind == kNib, "prefill GEMM: 4-bit (CQ4 / CQ3) codes only");
    ND_CHECK(geom.group >= 8, "prefill GEMM: groups of 8 or more");
    GemmArgs g{};
    g.xf = xf;
    g.codes = codes;
    g.norms = norms;
    g.y = y;
    g.m = m;
    g.rb_count = (m + 31) / 32;
    g.rows = rows;
    g.chunks = geom.chunks;
    g.groups = geom.groups;
    g.group_shift = __builtin_ctz(static_cast<unsigned>(geom.group));
    g.xsteps = dev / kBK;
    g.ksteps = (padded + kBK - 1) / kBK;  // dev is a multiple of 256: whole steps stay in the row
    g.mtiles = (m + kBM - 1) / kBM;
    g.tiles = (rows + kBN - 1) / kBN * g.mtiles;
    for (int q = 0; q < 4; ++q) {
        g.lo[q] = g.hi[q] = 0;
        for (int b = 0; b < 4; ++b) {
            g.lo[q] |= uint32_t(cb_half[q * 4 + b] & 0xFF) << (8 * b);
            g.hi[q] |= uint32_t(cb_half[q * 4 + b] >> 8) << (8 * b);
        }
    }
    dim3 grid(g.tiles), block(kGemmThreads);
    switch (g.group_shift) {
    case 3: hipLaunchKernelGGL(prefill_gemm_kernel<4>, grid, block, 0, s, g); break;
    case 4: hipLaunchKernelGGL(prefill_gemm_kernel<2>, grid, block, 0, s, g); break;
    default: hipLaunchKernelGGL(prefill_gemm_kernel<1>, grid, block, 0, s, g); break;
    }
    ND_HIP(hipGetLastError());
}

}  // namespace nd
