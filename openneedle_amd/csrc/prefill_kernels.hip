// gfx950 prefill GEMM: Y[m][n] = sum_k FWHT(X)[m][k] * cb[code[n][k]] * norm[n][k / group]
// on fp16 MFMA with fp32 accumulation (the batched form of cq.cpp:157-197,
// as Engine::linear_batch uses it for prompt chunks, engine.cpp:607-670).
//
// 1. prefill_transform_wave_kernel (groups <= 64: FWHT in registers and lane
//    butterflies) / prefill_transform_kernel (larger groups: FWHT in LDS):
//    per-group FWHT of X (the reference's stage order, then * 1/sqrt(group))
//    written as fp16 in MFMA fragment order:
//    each 16-byte slice is one lane's operand of one v_mfma_f32_32x32x16_f16,
//    so the GEMM loads X fragments straight from memory (1 KiB per wave load).
// 2. prefill_gemm_kernel: 128 x 128 output tile per workgroup, K in steps of
//    64 positions, two kinds of waves. Waves 0-3 (one per SIMD) each own 64
//    rows x 128 columns over half of the 16-position slices of every step
//    (the two K halves are summed through LDS at the end): X fragments from
//    memory two steps ahead, each loaded once per workgroup; weight fragments
//    from LDS, each read by two waves; 16 MFMAs per step. Waves 4-7 (one per SIMD) load
//    the 4-bit codes five steps ahead and dequantize the 128 x 64 weight
//    tile two steps ahead into a ring of three LDS buffers: codes -> fp16
//    codebook values times the fp16 group norm. One barrier per step; on each
//    SIMD the dequantization VALU work issues while the MFMA wave's matrix
//    instructions run. Tiles are ordered so that the
//    M-tiles of one N-tile run on the same XCD and share its L2. The
//    codebook lookup reads a 256-entry table of code pairs (two fp16 values
//    per byte of codes) from LDS, one private column per lane so the reads
//    are conflict-free: 4 v_perm + 4 ds_read_b32 + 4 v_pk_mul_f16 per 8 codes.
//
// 2-bit (CQ2, ternary) matrices are widened once to 4-bit device codes of the
// same positions (widen_crumbs_kernel), so one kernel serves every width.
//
// Rounding: X and the weights cb*norm are fp16 (two roundings for the
// weight), products and sums are fp32 in the MFMA; the result agrees with the
// reference FP32 path to about 1e-3 normwise (bound 2e-3).
#include "common.h"
#include "wave.h"

#include <hip/hip_fp16.h>

namespace nd {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kGemmThreads = 512;  // waves 0-3: MFMA (64 rows x 128 columns x half of K each); 4-7: dequantization
constexpr int kLdsRow = 72;        // halves per LDS weight row: 64 + 8 padding (conflict-free 16-byte accesses)
constexpr int kFragBytes = 1024;   // one operand fragment: 64 lanes x 8 halves
constexpr int kStepBytes = 4 * kFragBytes;  // the four 16-position slices of one 64-position step

// FWHT as transform_kernel, fp16 output in fragment order: for 32-row block
// rb, step s and slice kk, lane l holds row 32 rb + l % 32 and positions
// 64 s + 32 (l / 32) + 8 kk + e, e = 0..7. Rows m .. m32 - 1 are written as zeros.
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
            const int c0 = 2 * q, c1 = 2 * q + 1;
            const _Float16 h0 = static_cast<_Float16>(p0 + c0 < padded ? buf[8 * u + c0] * scale : 0.0f);
            const _Float16 h1 = static_cast<_Float16>(p0 + c1 < padded ? buf[8 * u + c1] * scale : 0.0f);
            w[q] = uint32_t(__builtin_bit_cast(uint16_t, h0)) | (uint32_t(__builtin_bit_cast(uint16_t, h1)) << 16);
        }
        const int s = p0 >> 6, hh = (p0 >> 5) & 1, kk = (p0 >> 3) & 3;
        const size_t idx = (((block + s) * 4 + kk) * 64 + hh * 32 + (v & 31)) * 8;
        *reinterpret_cast<u32x4 *>(xf + idx) = u32x4{w[0], w[1], w[2], w[3]};
    }
}

// Groups of 8 .. 64: one workgroup per (32-row block, 64-position step),
// thread (row r, unit u) = lane 8 (r % 8) + u owns positions 64 s + 8 u .. + 8
// of row r. FWHT stages 1, 2, 4 run on the thread's eight values, stages 8,
// 16, 32 are lane butterflies at strides 1, 2, 4 (the reference's stage order
// and operands, as transform_kernel); the thread writes its 16-byte slice of
// the fragment layout (eight rows of a wave: 128 contiguous bytes per slice).
template <int GROUP>
__global__ __launch_bounds__(256) void prefill_transform_wave_kernel(const float *__restrict__ x, int m, int in,
                                                                     int padded, int dev, float scale,
                                                                     _Float16 *__restrict__ xf) {
    static_assert(GROUP >= 8 && GROUP <= 64, "in-wave FWHT");
    const int s = blockIdx.x, rb = blockIdx.y;
    const int t = threadIdx.x, u = t & 7, r = t >> 3;  // r: row in the block (0..31)
    const int v = rb * 32 + r, p0 = s * kBK + 8 * u;
    float a[8];
    if (v < m && p0 + 8 <= in) {
        const float4 *src = reinterpret_cast<const float4 *>(x + static_cast<size_t>(v) * in + p0);
        if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
            const float4 lo = src[0], hi = src[1];
            a[0] = lo.x, a[1] = lo.y, a[2] = lo.z, a[3] = lo.w, a[4] = hi.x, a[5] = hi.y, a[6] = hi.z, a[7] = hi.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = x[static_cast<size_t>(v) * in + p0 + e];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = v < m && p0 + e < in ? x[static_cast<size_t>(v) * in + p0 + e] : 0.0f;
    }
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (!(e & h)) {
                const float lo = a[e], hi = a[e + h];
                a[e] = lo + hi;
                a[e + h] = lo - hi;
            }
#pragma unroll
    for (int e = 0; e < 8; ++e) wave_butterflies<GROUP / 8, 1>(a[e], t);
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const _Float16 h0 = static_cast<_Float16>(p0 + 2 * q < padded ? a[2 * q] * scale : 0.0f);
        const _Float16 h1 = static_cast<_Float16>(p0 + 2 * q + 1 < padded ? a[2 * q + 1] * scale : 0.0f);
        w[q] = uint32_t(__builtin_bit_cast(uint16_t, h0)) | (uint32_t(__builtin_bit_cast(uint16_t, h1)) << 16);
    }
    const int kk = u & 3, hh = u >> 2;
    const size_t idx = (((static_cast<size_t>(rb) * (dev / kBK) + s) * 4 + kk) * 64 + hh * 32 + r) * 8;
    *reinterpret_cast<u32x4 *>(xf + idx) = u32x4{w[0], w[1], w[2], w[3]};
}

// Code-pair table in LDS: entry e (a byte of codes: low nibble first) holds
// fp16 cb[e & 15] | cb[e >> 4] << 16. Each lane reads its own column (dword
// 64 e + lane), so a wave's 64 lookups hit 64 different banks.
constexpr int kPairEntries = 256;
constexpr int kPairWords = kPairEntries * 64;

struct GemmArgs {
    const _Float16 *xf;  // X in fragment order (prefill_transform_kernel), rb_count blocks of 32 rows
    const uint4 *codes;  // matrix device layout (4-bit codes)
    const uint16_t *norms;
    float *y;  // [m][rows]
    int m, rb_count, rows, chunks, groups, group_shift, xsteps, ksteps, mtiles, tiles;
    uint16_t cb[16];  // fp16 codebook
};

// Tile of this workgroup. Workgroups go to the 8 XCDs round robin; giving
// each XCD a contiguous run of tiles (M-tile fastest) keeps the M-tiles of an
// N-tile, which read the same codes, on one XCD's L2.
__device__ __forceinline__ int gemm_tile(const GemmArgs &g) {
    const int b = blockIdx.x;
    return g.tiles % 8 ? b : (b & 7) * (g.tiles >> 3) + (b >> 3);
}

// ---- MFMA waves ----------------------------------------------------------
// Wave (mi, ki) = (wave / 2, wave % 2) owns rows 64 mi .. + 64 and all 128
// columns of the tile over slices kk = 2 ki, 2 ki + 1 of every step (half of
// K): every X fragment is loaded once per workgroup and every weight
// fragment is read by two waves (the vector L1 delivers about a quarter of
// the LDS bandwidth, and LDS is shared with the dequantization waves).

struct AFrags {
    u32x4 v[2][2];  // [32-row block i][slice kk - 2 ki]
};

struct APtrs {
    __amdgpu_buffer_rsrc_t x;
    uint32_t xv[2];  // lane offsets of the wave's two row blocks (slice 2 ki)
};

__device__ __forceinline__ APtrs a_ptrs(const GemmArgs &g, int rb0, int ki, int lane) {
    const uint32_t block = static_cast<uint32_t>(g.xsteps) * kStepBytes;
    // blocks past the last read zero (scalar: a VALU clamp would make the descriptor divergent)
    const int live = __builtin_amdgcn_readfirstlane(min(2, max(0, g.rb_count - rb0)));
    APtrs p;
    p.x = buffer_rsrc(g.xf + static_cast<size_t>(rb0) * g.xsteps * (kStepBytes / 2), live * block);
    p.xv[0] = lane * 16u + ki * 2 * kFragBytes;
    p.xv[1] = p.xv[0] + block;
    return p;
}

__device__ __forceinline__ void a_load(AFrags &a, const APtrs &p, int s) {
    const int so = __builtin_amdgcn_readfirstlane(s * kStepBytes);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int k = 0; k < 2; ++k)
            a.v[i][k] = __builtin_amdgcn_raw_buffer_load_b128(p.x, p.xv[i] + k * kFragBytes, so, 0);
}

// Weight fragments of one slice for the four 32-column blocks: lane l holds
// weight row l % 32 of block j, slice kk of chunk l / 32.
struct BSlice {
    h8 v[4];
};

__device__ __forceinline__ void b_slice(BSlice &b, const _Float16 *Bs, int kk, int lane) {
    const _Float16 *B = Bs + (lane & 31) * kLdsRow + (lane >> 5) * 32 + kk * 8;
#pragma unroll
    for (int j = 0; j < 4; ++j) b.v[j] = *reinterpret_cast<const h8 *>(B + j * 32 * kLdsRow);
}

__device__ __forceinline__ void mma_slice(const AFrags &x, const BSlice &b, int k, f16x (&acc)[2][4]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8, x.v[i][k]), b.v[j], acc[i][j], 0,
                                                               0, 0);
}

// One K step of an MFMA wave (J = c % 6): X fragments of step c + 2 are
// requested (ring of three register sets); each slice's weight fragments are
// read one slice ahead of its MFMAs (the first slice of step c + 1 from LDS
// buffer (c + 1) % 3, complete since the previous barrier), so LDS latency
// hides behind eight MFMAs. Scheduling barriers keep the reads where they are.
template <int J>
__device__ __forceinline__ void mma_step(AFrags (&a)[3], BSlice (&b)[2], const GemmArgs &g, const APtrs &p, int c,
                                         const _Float16 (&Bs)[3][kBN * kLdsRow], f16x (&acc)[2][4], int ki,
                                         int lane) {
    a_load(a[(J + 2) % 3], p, min(c + 2, g.ksteps - 1));  // clamped: past the end it repeats the last step
    b_slice(b[1], Bs[J % 3], 2 * ki + 1, lane);
    __builtin_amdgcn_sched_barrier(0);
    mma_slice(a[J % 3], b[0], 0, acc);
    __builtin_amdgcn_sched_barrier(0);
    b_slice(b[0], Bs[(J + 1) % 3], 2 * ki, lane);  // past the end: never used
    __builtin_amdgcn_sched_barrier(0);
    mma_slice(a[J % 3], b[1], 1, acc);
    __builtin_amdgcn_sched_barrier(0);
    // Barrier without draining the four prefetch reads: LDS reads complete in
    // order, so lgkmcnt(4) retires every read of buffer c % 3 (rewritten in
    // step c + 1) while the reads of buffer (c + 1) % 3 (rewritten in step
    // c + 2) stay in flight. This wave writes no LDS.
    asm volatile("s_waitcnt lgkmcnt(4)\n\ts_barrier" ::: "memory");
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

// Code-pair lookups of one (weight row, chunk) of a step: 32 codes -> 16
// dwords of two fp16 codebook values, positions in order.
template <int NG>
__device__ __forceinline__ void table_reads(uint32_t (&v)[16], const CodeRegs<NG> &r, const uint32_t *pairs,
                                            uint32_t lane4) {
    const uint32_t c[4] = {r.code.x, r.code.y, r.code.z, r.code.w};
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // byte offset 256 * (byte k of code dword q) + 4 * lane: one v_perm (selector 0x0c gives zero bytes)
            const uint32_t off = __builtin_amdgcn_perm(c[q], lane4, 0x0c0c0400u + (k << 8));
            v[q * 4 + k] = *reinterpret_cast<const uint32_t *>(reinterpret_cast<const char *>(pairs) + off);
        }
}

// The looked-up values times the fp16 group norm -> LDS slots 32 ch .. + 32
// of weight row `row`.
template <int NG>
__device__ __forceinline__ void scale_store(const uint32_t (&v)[16], const CodeRegs<NG> &r, _Float16 *Bs, int row,
                                            int ch) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    u32x4 *d = reinterpret_cast<u32x4 *>(Bs + row * kLdsRow + ch * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t nm = r.norm[q * NG / 4];
        const h2 n = __builtin_bit_cast(h2, nm | (nm << 16));
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, v[q * 4 + k]) * n);
        d[q] = u32x4{w[0], w[1], w[2], w[3]};
    }
}

// Barrier of the dequantization waves. The last 16 LDS operations of the step
// are table reads issued after its four weight writes; LDS operations
// complete in order, so lgkmcnt(15) retires the writes (read by the MFMA
// waves after this barrier) and leaves the reads in flight across it.
__device__ __forceinline__ void deq_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(15)\n\ts_barrier" ::: "memory");
}

// One K step of a dequantization wave (J = c % 6): codes of step c + 5 are
// requested (ring of six), the table values of step c + 2 (read during step
// c - 1) are scaled into LDS buffer (c + 2) % 3, which the MFMA waves last
// read during step c - 1, and the table reads of step c + 3 are issued, so
// their latency hides behind a whole step.
template <int NG, int J>
__device__ __forceinline__ void deq_step(CodeRegs<NG> (&r)[6], uint32_t (&v)[16], const GemmArgs &g,
                                         const DPtrs &p, int c, const uint32_t *pairs, uint32_t lane4,
                                         _Float16 (&Bs)[3][kBN * kLdsRow], int row, int ch) {
    code_load(r[(J + 5) % 6], g, p, min(c + 5, g.ksteps - 1));
    if (c + 2 < g.ksteps) scale_store(v, r[(J + 2) % 6], Bs[(J + 2) % 3], row, ch);
    table_reads(v, r[(J + 3) % 6], pairs, lane4);  // past the end: clamped codes, never stored
    deq_barrier();
}

// Row block I of an MFMA wave's accumulators -> its slots of the park area
// (lane-interleaved 16-byte vectors, conflict-free).
template <int I>
__device__ __forceinline__ void park_block(const f16x (&acc)[2][4], u32x4 *park) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            park[((I * 4 + j) * 4 + q) * 64] = __builtin_bit_cast(
                u32x4, f32x4{acc[I][j][4 * q], acc[I][j][4 * q + 1], acc[I][j][4 * q + 2], acc[I][j][4 * q + 3]});
}

// Row block I (rows m_base + 32 I ..) of the tile: own partial sums plus the
// parked ones of the other K half, stored to Y.
template <int I>
__device__ __forceinline__ void store_block(const f16x (&acc)[2][4], const u32x4 *park, const GemmArgs &g,
                                            int m_base, int n0, int lane) {
    // C fragment: lane l holds column l % 32, rows 8 (e / 4) + 4 (l / 32) + e % 4
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + j * 32 + (lane & 31);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 o = __builtin_bit_cast(f32x4, park[((I * 4 + j) * 4 + q) * 64]);
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
                const int e = 4 * q + e4;
                const int m = m_base + I * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (n < g.rows && m < g.m) g.y[static_cast<size_t>(m) * g.rows + n] = acc[I][j][e] + o[e4];
            }
        }
    }
}

template <int NG>
__global__ __launch_bounds__(kGemmThreads) void prefill_gemm_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) _Float16 Bs[3][kBN * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint32_t pairs[kPairWords];
    // all 512 threads fill the code-pair table (16 x 16-byte stores each)
    for (int i = threadIdx.x; i < kPairWords / 4; i += kGemmThreads) {
        const int e = i >> 4;  // 16 vectors of 4 lanes per entry
        const uint32_t v = uint32_t(g.cb[e & 15]) | (uint32_t(g.cb[e >> 4]) << 16);
        reinterpret_cast<u32x4 *>(pairs)[i] = u32x4{v, v, v, v};
    }
    __syncthreads();
    const int tile = gemm_tile(g);
    const int n0 = (tile / g.mtiles) * kBN, m0 = (tile % g.mtiles) * kBM;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int last = g.ksteps - 1;
    // Every step ends in one barrier on both sides; the loops run in sixes so
    // that every ring index is a compile-time constant.
    if (wave < 4) {
        const int mi = wave >> 1, ki = wave & 1;
        const APtrs p = a_ptrs(g, m0 / 32 + 2 * mi, ki, lane);
        f16x acc[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = f16x{};
        AFrags a[3];
        BSlice b[2];
        a_load(a[0], p, 0);
        a_load(a[1], p, min(1, last));
        __syncthreads();  // weights of steps 0 and 1 are in LDS
        b_slice(b[0], Bs[0], 2 * ki, lane);
        int c = 0;
        for (; c + 6 <= g.ksteps; c += 6) {
            mma_step<0>(a, b, g, p, c, Bs, acc, ki, lane);
            mma_step<1>(a, b, g, p, c + 1, Bs, acc, ki, lane);
            mma_step<2>(a, b, g, p, c + 2, Bs, acc, ki, lane);
            mma_step<3>(a, b, g, p, c + 3, Bs, acc, ki, lane);
            mma_step<4>(a, b, g, p, c + 4, Bs, acc, ki, lane);
            mma_step<5>(a, b, g, p, c + 5, Bs, acc, ki, lane);
        }
        if (c < g.ksteps) mma_step<0>(a, b, g, p, c, Bs, acc, ki, lane);
        if (c + 1 < g.ksteps) mma_step<1>(a, b, g, p, c + 1, Bs, acc, ki, lane);
        if (c + 2 < g.ksteps) mma_step<2>(a, b, g, p, c + 2, Bs, acc, ki, lane);
        if (c + 3 < g.ksteps) mma_step<3>(a, b, g, p, c + 3, Bs, acc, ki, lane);
        if (c + 4 < g.ksteps) mma_step<4>(a, b, g, p, c + 4, Bs, acc, ki, lane);
        // Sum of the two K halves: each wave parks the row block that the
        // other half stores (over the code-pair table, no longer read), then
        // adds the parked partial sums to its own block (a two-term fp32 sum,
        // the same whichever side adds) and stores it: all four MFMA waves
        // store one 32-row block each.
        u32x4 *park = reinterpret_cast<u32x4 *>(pairs) + mi * 32 * 64 + lane;
        if (ki == 0) park_block<1>(acc, park);
        else park_block<0>(acc, park);
        __syncthreads();
        if (ki == 0) store_block<0>(acc, park, g, m0 + mi * 64, n0, lane);
        else store_block<1>(acc, park, g, m0 + mi * 64, n0, lane);
    } else {
        const int u = threadIdx.x - 256;
        const int row = u & (kBN - 1), ch = u >> 7;  // weight row of the tile, chunk of the step
        const DPtrs p = d_ptrs<NG>(g, n0, row, ch);
        const uint32_t lane4 = lane * 4u;
        CodeRegs<NG> r[6];
        uint32_t v[16];
#pragma unroll
        for (int k = 0; k < 5; ++k) code_load(r[k], g, p, min(k, last));
        table_reads(v, r[0], pairs, lane4);
        scale_store(v, r[0], Bs[0], row, ch);
        table_reads(v, r[1], pairs, lane4);
        if (1 < g.ksteps) scale_store(v, r[1], Bs[1], row, ch);
        table_reads(v, r[2], pairs, lane4);
        deq_barrier();
        int c = 0;
        for (; c + 6 <= g.ksteps; c += 6) {
            deq_step<NG, 0>(r, v, g, p, c, pairs, lane4, Bs, row, ch);
            deq_step<NG, 1>(r, v, g, p, c + 1, pairs, lane4, Bs, row, ch);
            deq_step<NG, 2>(r, v, g, p, c + 2, pairs, lane4, Bs, row, ch);
            deq_step<NG, 3>(r, v, g, p, c + 3, pairs, lane4, Bs, row, ch);
            deq_step<NG, 4>(r, v, g, p, c + 4, pairs, lane4, Bs, row, ch);
            deq_step<NG, 5>(r, v, g, p, c + 5, pairs, lane4, Bs, row, ch);
        }
        if (c < g.ksteps) deq_step<NG, 0>(r, v, g, p, c, pairs, lane4, Bs, row, ch);
        if (c + 1 < g.ksteps) deq_step<NG, 1>(r, v, g, p, c + 1, pairs, lane4, Bs, row, ch);
        if (c + 2 < g.ksteps) deq_step<NG, 2>(r, v, g, p, c + 2, pairs, lane4, Bs, row, ch);
        if (c + 3 < g.ksteps) deq_step<NG, 3>(r, v, g, p, c + 3, pairs, lane4, Bs, row, ch);
        if (c + 4 < g.ksteps) deq_step<NG, 4>(r, v, g, p, c + 4, pairs, lane4, Bs, row, ch);
        __syncthreads();  // the MFMA waves' K-half exchange
    }
}

}  // namespace

size_t prefill_xf_halves(int m, int dev) { return static_cast<size_t>((m + 31) / 32) * 32 * dev; }

void launch_prefill_transform(const float *x, int m, int in, int padded, int dev, int group, float scale,
                              _Float16 *xf, hipStream_t s) {
    if (m <= 0) return;
    ND_CHECK(group <= 16384, "prefill GEMM: group must be <= 16384");
    ND_CHECK(dev % kBK == 0, "internal: prefill rows must be whole 64-position steps");
    if (group <= 64) {
        dim3 grid(dev / kBK, (m + 31) / 32), block(256);
        switch (group) {
        case 8: hipLaunchKernelGGL(prefill_transform_wave_kernel<8>, grid, block, 0, s, x, m, in, padded, dev, scale, xf); break;
        case 16: hipLaunchKernelGGL(prefill_transform_wave_kernel<16>, grid, block, 0, s, x, m, in, padded, dev, scale, xf); break;
        case 32: hipLaunchKernelGGL(prefill_transform_wave_kernel<32>, grid, block, 0, s, x, m, in, padded, dev, scale, xf); break;
        default: hipLaunchKernelGGL(prefill_transform_wave_kernel<64>, grid, block, 0, s, x, m, in, padded, dev, scale, xf); break;
        }
        ND_HIP(hipGetLastError());
        return;
    }
    const int seg = group > 1024 ? group : 1024;
    dim3 grid((dev + seg - 1) / seg, (m + 31) / 32 * 32), block(256);
    hipLaunchKernelGGL(prefill_transform_kernel, grid, block, seg * sizeof(float), s, x, m, in, padded, dev, group,
                       scale, xf, seg);
    ND_HIP(hipGetLastError());
}

void launch_prefill_gemm(const CqGeom &geom, const uint4 *codes4, int chunks4, const uint16_t *norms, int rows,
                         const _Float16 *xf, int m, int dev, int padded, const uint16_t *cb_half, float *y,
                         hipStream_t s) {
    if (m <= 0) return;
    ND_CHECK(geom.group >= 8, "prefill GEMM: groups of 8 or more");
    ND_CHECK(chunks4 * 32 == dev, "internal: prefill GEMM takes 4-bit codes (32 per chunk)");
    GemmArgs g{};
    g.xf = xf;
    g.codes = codes4;
    g.norms = norms;
    g.y = y;
    g.m = m;
    g.rb_count = (m + 31) / 32;
    g.rows = rows;
    g.chunks = chunks4;
    g.groups = geom.groups;
    g.group_shift = __builtin_ctz(static_cast<unsigned>(geom.group));
    g.xsteps = dev / kBK;
    g.ksteps = (padded + kBK - 1) / kBK;  // dev is a multiple of 256: whole steps stay in the row
    g.mtiles = (m + kBM - 1) / kBM;
    g.tiles = (rows + kBN - 1) / kBN * g.mtiles;
    for (int i = 0; i < 16; ++i) g.cb[i] = cb_half[i];
    dim3 grid(g.tiles), block(kGemmThreads);
    switch (g.group_shift) {
    case 3: hipLaunchKernelGGL(prefill_gemm_kernel<4>, grid, block, 0, s, g); break;
    case 4: hipLaunchKernelGGL(prefill_gemm_kernel<2>, grid, block, 0, s, g); break;
    default: hipLaunchKernelGGL(prefill_gemm_kernel<1>, grid, block, 0, s, g); break;
    }
    ND_HIP(hipGetLastError());
}

namespace {

// 2-bit device codes -> 4-bit device codes of the same positions (crumb i of
// a byte becomes nibble i): the prefill GEMM's input for CQ2 and ternary
// matrices. One thread per (row tile, 32-position chunk, row).
__global__ __launch_bounds__(256) void widen_crumbs_kernel(const uint4 *__restrict__ src, int chunks2,
                                                           uint4 *__restrict__ dst, int chunks4) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    const int row = static_cast<int>(idx % kRowsPerBlock);
    const size_t tc = idx / kRowsPerBlock;
    const int c4 = static_cast<int>(tc % chunks4);
    const size_t tile = tc / chunks4;
    const uint4 in = src[(tile * chunks2 + c4 / 2) * kRowsPerBlock + row];
    const uint32_t half[2] = {(c4 & 1) ? in.z : in.x, (c4 & 1) ? in.w : in.y};  // bytes 8 (c4 % 2) .. + 8
    uint32_t out[4];
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            uint32_t r = 0;
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const uint32_t byte = (half[d] >> (8 * (2 * k + b))) & 0xFFu;
                const uint32_t nib = (byte & 3u) | ((byte >> 2) & 3u) << 4 | ((byte >> 4) & 3u) << 8 |
                                     ((byte >> 6) & 3u) << 12;
                r |= nib << (16 * b);
            }
            out[2 * d + k] = r;
        }
    dst[idx] = uint4{out[0], out[1], out[2], out[3]};
}

}  // namespace

void launch_widen_crumbs(const uint4 *codes2, int chunks2, int n_pad, uint4 *codes4, hipStream_t s) {
    const int chunks4 = 2 * chunks2;
    const size_t total = static_cast<size_t>(n_pad) * chunks4;  // n_pad is a multiple of 256
    hipLaunchKernelGGL(widen_crumbs_kernel, dim3(static_cast<unsigned>(total / 256)), dim3(256), 0, s, codes2, chunks2,
                       codes4, chunks4);
    ND_HIP(hipGetLastError());
}

}  // namespace nd
