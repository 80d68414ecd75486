// gfx950 prefill GEMM: Y[m][n] = sum_k FWHT(X)[m][k] * cb[code[n][k]] * norm[n][k / group]
// on fp16 MFMA with fp32 accumulation (the batched form of cq.cpp:157-197,
// as Engine::linear_batch uses it for prompt chunks, engine.cpp:607-670).
//
// 1. prefill_transform_kernel: per-group FWHT of X (the reference's stage
//    order, then * 1/sqrt(group)) written as fp16, rows of `dev` halves.
// 2. prefill_gemm_kernel: 128 x 128 output tile per workgroup, 4 waves in a
//    2 x 2 arrangement of 64 x 64 (2 x 2 v_mfma_f32_32x32x16_f16 tiles), K in
//    steps of 64 positions. Per step the X tile (128 x 64 fp16) is staged in
//    LDS and the 128 x 64 weight tile is dequantized once per workgroup into
//    LDS: 4-bit codes -> fp16 codebook values through v_perm byte tables,
//    times the fp16 group norm (v_pk_mul_f16). Global loads run three steps
//    ahead through a ring of four register sets; LDS is double-buffered.
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
constexpr int kLdsRow = 72;  // halves per LDS row: 64 + 8 padding (conflict-free 16-byte fragment reads)

// Same FWHT as transform_kernel, fp16 output (cast after the fp32 scale).
__global__ __launch_bounds__(256) void prefill_transform_kernel(const float *__restrict__ x, int in, int padded,
                                                                int dev, int group, float scale,
                                                                _Float16 *__restrict__ out, int seg) {
    extern __shared__ float buf[];
    const int v = blockIdx.y;
    const int base = blockIdx.x * seg;
    const float *xv = x + static_cast<size_t>(v) * in;
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
    // stored in the GEMM's K order: positions 0,2,4,6,1,3,5,7 of each 8
    _Float16 *ov = out + static_cast<size_t>(v) * dev;
    for (int i = threadIdx.x; i < seg; i += blockDim.x) {
        const int p = base + i;
        if (p < dev) ov[(p & ~7) | ((p & 1) << 2) | ((p & 7) >> 1)] = static_cast<_Float16>(p < padded ? buf[i] * scale : 0.0f);
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
// (both halves of `norm2`), in the GEMM's K order 0,2,4,6,1,3,5,7 (the
// activations are stored in the same order), which saves re-interleaving.
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
    const _Float16 *xh;   // [m][dev], K order permuted within each 8 (prefill_transform_kernel)
    const uint4 *codes;   // matrix device layout (4-bit codes)
    const uint16_t *norms;
    float *y;             // [m][rows]
    int m, rows, dev, chunks, groups, group_shift, ksteps;
    uint32_t lo[4], hi[4];  // fp16 codebook, low / high byte tables
};

// Buffer resources and per-thread offsets of one workgroup; every per-step
// offset is wave-uniform (soffset), so loads cost no address arithmetic.
struct GemmPtrs {
    __amdgpu_buffer_rsrc_t x, c, n;
    uint32_t xv, cv, nv[4];  // per-thread voffsets: X row, code chunk, the four norm dwords
    int nshift;              // norm soffset per step: (ks * 64) >> group_shift groups (or ks * (64 >> shift))
};

__device__ __forceinline__ GemmPtrs gemm_ptrs(const GemmArgs &g, int m0, int n0) {
    const int t = threadIdx.x;
    const int row = t >> 1, half = t & 1;
    GemmPtrs p;
    const int mrows = min(kBM, g.m - m0);  // rows past m are outside the buffer and read zero
    p.x = buffer_rsrc(g.xh + static_cast<size_t>(m0) * g.dev, static_cast<uint32_t>(mrows) * g.dev * 2u);
    p.xv = (static_cast<uint32_t>(row) * g.dev + half * 32) * 2u;
    const int tile = n0 / kRowsPerBlock, r = n0 % kRowsPerBlock + row;  // row inside its 256-row tile
    p.c = buffer_rsrc(g.codes + static_cast<size_t>(tile) * g.chunks * kRowsPerBlock,
                      static_cast<uint32_t>(g.chunks) * kRowsPerBlock * 16u);
    p.cv = (static_cast<uint32_t>(half) * kRowsPerBlock + r) * 16u;
    // groups past the last (positions past `padded`) read zero through the bound
    p.n = buffer_rsrc(g.norms + static_cast<size_t>(tile) * g.groups * kRowsPerBlock,
                      static_cast<uint32_t>(g.groups) * kRowsPerBlock * 2u);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int q = half * 32 + j * 8;  // position of code dword j inside the 64-position step
        const int gq = g.group_shift <= 6 ? q >> g.group_shift : 0;
        p.nv[j] = (static_cast<uint32_t>(gq) * kRowsPerBlock + r) * 2u;
    }
    return p;
}

// Global -> register staging of one K step (64 positions): thread t owns
// row t / 2, positions 32 (t % 2) .. + 32 of both the X tile and the weight
// tile (one 16-byte code chunk).
struct StepRegs {
    u32x4 a[4];        // 32 halves of one X row
    u32x4 code;        // 32 codes of one weight row
    uint32_t norm[4];  // fp16 norm bits of the four code dwords
};

// Loaded values stay raw (no ALU work on in-flight loads here).
__device__ __forceinline__ void gemm_load(StepRegs &r, const GemmArgs &g, const GemmPtrs &p, int ks) {
    // X: halves 64 ks + 32 half .. + 32 of this thread's row
#pragma unroll
    for (int q = 0; q < 4; ++q) r.a[q] = __builtin_amdgcn_raw_buffer_load_b128(p.x, p.xv, ks * kBK * 2 + q * 16, 0);
    // weights: chunk 2 ks + half of this thread's weight row
    r.code = __builtin_amdgcn_raw_buffer_load_b128(p.c, p.cv, ks * 2 * kRowsPerBlock * 16, 0);
    const int gs = g.group_shift <= 6 ? ks << (6 - g.group_shift) : (ks << 6) >> g.group_shift;  // step's first group
#pragma unroll
    for (int j = 0; j < 4; ++j)
        r.norm[j] = __builtin_amdgcn_raw_buffer_load_b16(p.n, p.nv[j], gs * kRowsPerBlock * 2, 0);
}

__device__ __forceinline__ void gemm_store(const StepRegs &r, const GemmArgs &g, _Float16 *As, _Float16 *Bs) {
    const int t = threadIdx.x;
    const int row = t >> 1, half = t & 1;
    u32x4 *ad = reinterpret_cast<u32x4 *>(As + row * kLdsRow + half * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) ad[q] = r.a[q];
    // Opaque here, so the dequantization is not hoisted above the step's
    // prefetch and MFMAs (where it would wait for these loads early).
    uint32_t c[4] = {r.code.x, r.code.y, r.code.z, r.code.w};
    uint32_t nm[4] = {r.norm[0], r.norm[1], r.norm[2], r.norm[3]};
    asm volatile("" : "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(nm[0]), "+v"(nm[1]), "+v"(nm[2]), "+v"(nm[3]));
    u32x4 *bd = reinterpret_cast<u32x4 *>(Bs + row * kLdsRow + half * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t w[4];
        dequant8(c[q], g.lo, g.hi, nm[q] | (nm[q] << 16), w);
        bd[q] = u32x4{w[0], w[1], w[2], w[3]};
    }
}

// One K step: its global loads were issued three steps earlier (ring of 4
// register sets), it is computed from LDS buffer c % 2 while step c + 1 is
// dequantized into the other buffer.
template <int J>
__device__ __forceinline__ void gemm_step(StepRegs (&r)[4], const GemmArgs &g, const GemmPtrs &p, int c,
                                          _Float16 (&As)[2][kBM * kLdsRow],
                                          _Float16 (&Bs)[2][kBN * kLdsRow], f16x (&acc)[2][2]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    gemm_load(r[(J + 3) & 3], g, p, min(c + 3, g.ksteps - 1));  // clamped: past the end it repeats the last step
    asm volatile("" ::: "memory");
    const _Float16 *A = As[c & 1];
    const _Float16 *B = Bs[c & 1];
    // operand fragments: lane l holds row l % 32, halves 8 (l / 32) .. + 8
    const int fr = lane & 31, fk = (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 16) {
        h8 af[2], bf[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const h8 *>(A + (wm * 64 + i * 32 + fr) * kLdsRow + kk + fk);
#pragma unroll
        for (int j = 0; j < 2; ++j) bf[j] = *reinterpret_cast<const h8 *>(B + (wn * 64 + j * 32 + fr) * kLdsRow + kk + fk);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    gemm_store(r[(J + 1) & 3], g, As[(c + 1) & 1], Bs[(c + 1) & 1]);  // past the end: never read
    __syncthreads();
}

__global__ __launch_bounds__(256) void prefill_gemm_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) _Float16 As[2][kBM * kLdsRow];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][kBN * kLdsRow];
    const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * kBM;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;  // this wave: rows 64 wm.., columns 64 wn..
    const GemmPtrs p = gemm_ptrs(g, m0, n0);

    f16x acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f16x{};

    StepRegs r[4];
    const int last = g.ksteps - 1;
    gemm_load(r[0], g, p, 0);
    gemm_load(r[1], g, p, min(1, last));
    gemm_load(r[2], g, p, min(2, last));
    gemm_store(r[0], g, As[0], Bs[0]);
    __syncthreads();
    int c = 0;
    for (; c + 4 <= g.ksteps; c += 4) {
        gemm_step<0>(r, g, p, c, As, Bs, acc);
        gemm_step<1>(r, g, p, c + 1, As, Bs, acc);
        gemm_step<2>(r, g, p, c + 2, As, Bs, acc);
        gemm_step<3>(r, g, p, c + 3, As, Bs, acc);
    }
    // 0 to 3 remaining steps (set indices continue the ring)
    if (c < g.ksteps) gemm_step<0>(r, g, p, c, As, Bs, acc);
    if (c + 1 < g.ksteps) gemm_step<1>(r, g, p, c + 1, As, Bs, acc);
    if (c + 2 < g.ksteps) gemm_step<2>(r, g, p, c + 2, As, Bs, acc);
    // C fragment: lane l holds column l % 32, rows 8 (e / 4) + 4 (l / 32) + e % 4
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= g.rows) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (m < g.m) g.y[static_cast<size_t>(m) * g.rows + n] = acc[i][j][e];
            }
        }
}

}  // namespace

void launch_prefill_transform(const float *x, int m, int in, int padded, int dev, int group, float scale,
                              _Float16 *xh, hipStream_t s) {
    if (m <= 0) return;
    ND_CHECK(group <= 16384, "prefill GEMM: group must be <= 16384");
    const int seg = group > 1024 ? group : 1024;
    dim3 grid((dev + seg - 1) / seg, m), block(256);
    hipLaunchKernelGGL(prefill_transform_kernel, grid, block, seg * sizeof(float), s, x, in, padded, dev, group, scale,
                       xh, seg);
    ND_HIP(hipGetLastError());
}

void launch_prefill_gemm(const CqGeom &geom, const uint4 *codes, const uint16_t *norms, int rows, const _Float16 *xh,
                         int m, int dev, int padded, const uint16_t *cb_half, float *y, hipStream_t s) {
    if (m <= 0) return;
    ND_CHECK(geom.kind == kNib, "prefill GEMM: 4-bit (CQ4 / CQ3) codes only");
    GemmArgs g{};
    g.xh = xh;
    g.codes = codes;
    g.norms = norms;
    g.y = y;
    g.m = m;
    g.rows = rows;
    g.dev = dev;
    g.chunks = geom.chunks;
    g.groups = geom.groups;
    g.group_shift = __builtin_ctz(static_cast<unsigned>(geom.group));
    g.ksteps = (padded + kBK - 1) / kBK;  // dev is a multiple of 256: whole steps stay in the row
    for (int q = 0; q < 4; ++q) {
        g.lo[q] = g.hi[q] = 0;
        for (int b = 0; b < 4; ++b) {
            g.lo[q] |= uint32_t(cb_half[q * 4 + b] & 0xFF) << (8 * b);
            g.hi[q] |= uint32_t(cb_half[q * 4 + b] >> 8) << (8 * b);
        }
    }
    dim3 grid((rows + kBN - 1) / kBN, (m + kBM - 1) / kBM), block(256);
    hipLaunchKernelGGL(prefill_gemm_kernel, grid, block, 0, s, g);
    ND_HIP(hipGetLastError());
}

}  // namespace nd
