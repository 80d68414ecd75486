// gfx950 kernels for the FP32 CQ path: device layout, activation FWHT,
// packed GEMV and row dequantization.
//
// GEMV design (decode, HBM-bound): one lane per output row. Codes are stored
// chunk-major (common.h) so a wavefront reads 1 KiB contiguous per 16-byte
// chunk step. The activation side becomes per-position product tables in LDS,
// rebuilt per 256-position window and shared by the workgroup's 256 rows, so
// each code costs one LDS read plus one add, in the reference's own order.
// All files are compiled with -ffp-contract=off.
#include "common.h"
#include "wave.h"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>

namespace nd {

namespace {

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

__device__ __forceinline__ float lds_at(const float *base, uint32_t byte_offset) {
    return *reinterpret_cast<const float *>(reinterpret_cast<const char *>(base) + byte_offset);
}

// ---------------------------------------------------------------------------
// Layout
// ---------------------------------------------------------------------------
__global__ void relayout_kernel(const uint8_t *__restrict__ packed, int rows, int rowbytes, int bits,
                                int padded, uint4 *__restrict__ codes, int n_pad, int chunks) {
    int r = blockIdx.x * blockDim.x + threadIdx.x;
    int c = blockIdx.y;
    if (r >= n_pad || c >= chunks) return;
    uint32_t out[4] = {0, 0, 0, 0};
    if (r < rows) {
        const uint8_t *row = packed + static_cast<size_t>(r) * rowbytes;
        if (bits == 3) {
            // widen LSB-first 3-bit codes to nibbles: positions 32c .. 32c+31
            for (int i = 0; i < 32; ++i) {
                int pos = c * 32 + i;
                if (pos >= padded) break;
                int bit = pos * 3, byte = bit >> 3, shift = bit & 7;
                unsigned word = row[byte];
                if (shift + 3 > 8) word |= unsigned(row[byte + 1]) << 8;
                unsigned code = (word >> shift) & 7u;
                out[i >> 3] |= code << ((i & 7) * 4);
            }
        } else {
            for (int i = 0; i < 16; ++i) {
                int byte = c * 16 + i;
                if (byte < rowbytes) out[i >> 2] |= uint32_t(row[byte]) << ((i & 3) * 8);
            }
        }
    }
    codes[code_index(r, c, chunks)] = make_uint4(out[0], out[1], out[2], out[3]);
}

__global__ void norms_transpose_kernel(const uint16_t *__restrict__ norms, int rows, int groups,
                                       uint16_t *__restrict__ out, int n_pad) {
    int r = blockIdx.x * blockDim.x + threadIdx.x;
    int g = blockIdx.y;
    if (r >= n_pad) return;
    out[norm_index(r, g, groups)] = r < rows ? norms[static_cast<size_t>(r) * groups + g] : uint16_t(0);
}

// ---------------------------------------------------------------------------
// FWHT per group (cq.cpp:30-46, 153-156). Each butterfly is the same
// (a+b, a-b) on the same operands as the sequential loop, stage h ascending,
// then one multiply by the host-computed float 1/sqrt(group): bit-exact.
// One block owns a segment of `seg` positions (a multiple of the group).
// Positions >= in are zero before the transform; positions in
// [padded, out_limit) are stored as zero.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void transform_kernel(const float *__restrict__ x, int x_stride,
                                                        float *__restrict__ rot, int rot_stride, int in,
                                                        int padded, int out_limit, int group, float scale,
                                                        int seg) {
    extern __shared__ float buf[];
    const int v = blockIdx.y;
    const int base = blockIdx.x * seg;
    const float *xv = x + static_cast<size_t>(v) * x_stride;
    float *rv = rot + static_cast<size_t>(v) * rot_stride;
    for (int i = threadIdx.x; i < seg; i += blockDim.x) {
        int p = base + i;
        buf[i] = p < in ? xv[p] : 0.0f;
    }
    __syncthreads();
    if (base < padded) {
        for (int h = 1; h < group; h <<= 1) {
            for (int t = threadIdx.x; t < seg / 2; t += blockDim.x) {
                int lo = (t / h) * 2 * h + (t % h);
                float a = buf[lo], b = buf[lo + h];
                buf[lo] = a + b;
                buf[lo + h] = a - b;
            }
            __syncthreads();
        }
    }
    for (int i = threadIdx.x; i < seg; i += blockDim.x) {
        int p = base + i;
        if (p < out_limit) rv[p] = p < padded ? buf[i] * scale : 0.0f;
    }
}

// Fallback for groups too large for one block's LDS: global-memory stages.
__global__ void pad_copy_kernel(const float *__restrict__ x, int x_stride, float *__restrict__ rot,
                                int rot_stride, int in, int n) {
    int p = blockIdx.x * blockDim.x + threadIdx.x;
    int v = blockIdx.y;
    if (p < n) rot[static_cast<size_t>(v) * rot_stride + p] = p < in ? x[static_cast<size_t>(v) * x_stride + p] : 0.0f;
}

__global__ void butterfly_stage_kernel(float *__restrict__ rot, int rot_stride, int padded, int h) {
    int t = blockIdx.x * blockDim.x + threadIdx.x;
    int v = blockIdx.y;
    if (t >= padded / 2) return;
    float *rv = rot + static_cast<size_t>(v) * rot_stride;
    int lo = (t / h) * 2 * h + (t % h);
    float a = rv[lo], b = rv[lo + h];
    rv[lo] = a + b;
    rv[lo + h] = a - b;
}

__global__ void scale_crop_kernel(const float *__restrict__ src, int src_stride, float *__restrict__ dst,
                                  int dst_stride, int padded, int out_limit, float scale) {
    int p = blockIdx.x * blockDim.x + threadIdx.x;
    int v = blockIdx.y;
    if (p < out_limit)
        dst[static_cast<size_t>(v) * dst_stride + p] =
            p < padded ? src[static_cast<size_t>(v) * src_stride + p] * scale : 0.0f;
}

// ---------------------------------------------------------------------------
// Packed FP32 GEMV
//
// Per 256-position window the workgroup builds a product table in LDS:
//   4-bit codes: slot p (one position), 16 floats  T[p][c]        = cb[c]*rot[p]
//   2-bit codes: slot s (two positions), 16 float2 T[s][c0|c1<<2] = (cb[c0]*rot[2s], cb[c1]*rot[2s+1])
// Each lane (one row) walks its codes in order: one LDS read per 4-bit code
// or per pair of 2-bit codes, then gd += product (sequentially, one add per
// code). Groups close with sum += gd * half(norm). This is the reference's
// exact operation sequence (cq.cpp:104-107, 157-164, 185-194) for every bit
// width, so results are bit-identical to its portable build.
//
// For groups up to one window the activation FWHT (cq.cpp:30-46, 153-156) is
// computed in the kernel from x: lane t owns position t of the window;
// butterflies of stride < 64 are wave shuffles, 64 and 128 go through LDS.
// Slot strides are padded (17 / 34 floats) so table writes are bank-conflict
// free; reads are wave-uniform per slot (broadcast).
// ---------------------------------------------------------------------------
template <int KIND>
struct TableShape {
    static constexpr int kCodesPerChunk = KIND == kNib ? 32 : 64;
    static constexpr int kChunksPerWindow = kWindow / kCodesPerChunk;
    static constexpr int kPositionsPerSlot = KIND == kNib ? 1 : 2;
    static constexpr int kSlots = kWindow / kPositionsPerSlot;     // slots per window
    static constexpr int kEntryBytes = KIND == kNib ? 4 : 8;
    static constexpr int kSlotFloats = KIND == kNib ? 17 : 36;     // 16 entries + padding
    static constexpr int kFloats = kSlots * kSlotFloats;
};

// Positions of a window handled by one thread: t, t + kRowsPerBlock, ...
constexpr int kPositionsPerThread = kWindow / kRowsPerBlock;

// Window activations: x (fused) or rot (precomputed) for this thread's
// positions, through a buffer resource bounded at the row's end, so positions
// >= in read as zero (the reference's zero padding, cq.cpp:154).
__device__ __forceinline__ void load_act(__amdgpu_buffer_rsrc_t act, int w, float (&a)[kPositionsPerThread]) {
#pragma unroll
    for (int k = 0; k < kPositionsPerThread; ++k)
        a[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             act, (k * kRowsPerBlock + threadIdx.x) * 4u, w * kWindow * 4, 0));
}

// In-kernel FWHT of the window (GROUP <= kWindow), identical butterflies to
// the reference (stage h ascending: (a+b, a-b)), then the multiply by the
// host-computed 1/sqrt(group). Strides below 64 are wave shuffles; larger
// strides exchange through LDS.
template <int GROUP>
__device__ __forceinline__ void window_fwht(float (&v)[kPositionsPerThread], float scale, float *stage) {
    const int t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < kPositionsPerThread; ++k) wave_butterflies<GROUP, 1>(v[k], t & 63);
    if constexpr (GROUP > 64) {
#pragma unroll
        for (int h = 64; h < GROUP; h <<= 1) {
#pragma unroll
            for (int k = 0; k < kPositionsPerThread; ++k) stage[k * kRowsPerBlock + t] = v[k];
            __syncthreads();
            float o[kPositionsPerThread];
#pragma unroll
            for (int k = 0; k < kPositionsPerThread; ++k) o[k] = stage[(k * kRowsPerBlock + t) ^ h];
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kPositionsPerThread; ++k) {
                const int p = k * kRowsPerBlock + t;
                const float sv = (p & h) ? -v[k] : v[k];
                v[k] = o[k] + sv;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kPositionsPerThread; ++k) v[k] = v[k] * scale;
}

// Write the window's products into the table. 4-bit: lane t fills slot t
// (stride 17 floats: conflict-free 4-byte writes). 2-bit: in each wave, lanes
// 0..31 fill slots for the wave's 64 positions, taking the two positions'
// values from their neighbours by shuffle (stride 36 floats, 16-byte writes).
template <int KIND>
__device__ __forceinline__ void build_table(float *__restrict__ T, const float *lut,
                                            const float (&r)[kPositionsPerThread]) {
    using S = TableShape<KIND>;
    const int t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < kPositionsPerThread; ++k) {
        if constexpr (KIND == kNib) {
            float *dst = T + (k * kRowsPerBlock + t) * S::kSlotFloats;
#pragma unroll
            for (int c = 0; c < 16; ++c) dst[c] = lut[c] * r[k];
        } else {
            const int lane = t & 63;
            const int l = lane & 31;
            const float r0 = __shfl(r[k], 2 * l);
            const float r1 = __shfl(r[k], 2 * l + 1);
            if (lane < 32) {
                float p0[4], p1[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    p0[c] = lut[c] * r0;
                    p1[c] = lut[c] * r1;
                }
                // entry n = c0 | c1 << 2 holds (p0[c0], p1[c1]); two entries per 16-byte store
                const int slot = (k * kRowsPerBlock + (t & ~63)) / 2 + l;
                float4 *dst = reinterpret_cast<float4 *>(T + slot * S::kSlotFloats);
#pragma unroll
                for (int hi = 0; hi < 4; ++hi) {
                    dst[2 * hi] = make_float4(p0[0], p1[hi], p0[1], p1[hi]);
                    dst[2 * hi + 1] = make_float4(p0[2], p1[hi], p0[3], p1[hi]);
                }
            }
        }
    }
}

// GROUP > 0: the group size, at most one window; GROUP == 0: group > kWindow
// (a group spans whole windows and closes at a window end).
template <int GROUP>
struct NormsPerWindow {
    static constexpr int value = GROUP > 0 ? kWindow / GROUP : 1;
};

template <int KIND, int GROUP>
struct WindowState {
    static constexpr int kChunks = TableShape<KIND>::kChunksPerWindow;
    static constexpr int kNorms = NormsPerWindow<GROUP>::value;
    u32x4 codes[kChunks];
    uint16_t norms[kNorms];
};

// Buffer loads from the workgroup's row tile: the chunk / group offset is
// wave-uniform (soffset) and the per-lane offset is one shared VGPR, so no
// per-chunk addresses stay live.
template <int KIND, int GROUP>
__device__ __forceinline__ void load_window(WindowState<KIND, GROUP> &st, __amdgpu_buffer_rsrc_t codes,
                                            __amdgpu_buffer_rsrc_t norms, int w, int groups, int windows_per_group) {
    constexpr int C = WindowState<KIND, GROUP>::kChunks;
    constexpr int NN = WindowState<KIND, GROUP>::kNorms;
    const uint32_t code_lane = threadIdx.x * 16u;
    const uint32_t norm_lane = threadIdx.x * 2u;
#pragma unroll
    for (int c = 0; c < C; ++c)
        st.codes[c] = __builtin_amdgcn_raw_buffer_load_b128(codes, code_lane, (w * C + c) * kRowsPerBlock * 16,
                                                             kStreamLoad);
    // group indices are clamped (phantom groups past the last are never closed)
    if constexpr (GROUP > 0) {
#pragma unroll
        for (int k = 0; k < NN; ++k) {
            const int g = min(w * NN + k, groups - 1);
            st.norms[k] = __builtin_amdgcn_raw_buffer_load_b16(norms, norm_lane, g * kRowsPerBlock * 2, 0);
        }
    } else {
        const int g = min(w / windows_per_group, groups - 1);
        st.norms[0] = __builtin_amdgcn_raw_buffer_load_b16(norms, norm_lane, g * kRowsPerBlock * 2, 0);
    }
}

// Byte offsets of the 8 slot entries addressed by one code dword: 8 nibbles,
// spread into X (even nibbles) and Y (odd nibbles), one v_bfe each.
template <int KIND>
__device__ __forceinline__ void slot_offsets(uint32_t wd, uint32_t off[8]) {
    constexpr int kShift = KIND == kNib ? 2 : 3;  // entry bytes: 4 or 8
    constexpr uint32_t kMask = KIND == kNib ? 0x3C3C3C3Cu : 0x78787878u;
    uint32_t X = (wd << kShift) & kMask;
    uint32_t Y = (wd >> (4 - kShift)) & kMask;
    // opaque to the optimizer: keeps one v_bfe per slot instead of a
    // re-derived shift+and pair
    asm("" : "+v"(X));
    asm("" : "+v"(Y));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t src = (i & 1) ? Y : X;
        const int sh = (i >> 1) * 8;
        off[i] = sh == 24 ? (src >> 24) : ((src >> sh) & 0xFFu);
    }
}

template <int KIND>
struct SlotValues {
    float a[8];
    float b[8];  // second code of a 2-bit pair
};

template <int KIND>
__device__ __forceinline__ void read_slots(const float *T, int slot0, const uint32_t off[8], SlotValues<KIND> &v) {
    using S = TableShape<KIND>;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const char *slot = reinterpret_cast<const char *>(T + (slot0 + i) * S::kSlotFloats);
        if constexpr (KIND == kNib) {
            v.a[i] = *reinterpret_cast<const float *>(slot + off[i]);
        } else {
            const float2 pr = *reinterpret_cast<const float2 *>(slot + off[i]);
            v.a[i] = pr.x;
            v.b[i] = pr.y;
        }
    }
}

#ifndef ND_PIPE
#define ND_PIPE 2
#endif
#ifndef ND_SCHED_BARRIER
#define ND_SCHED_BARRIER 1
#endif

// Process one window against its table T (LDS), in the reference's order.
// Software pipeline, fixed with scheduling barriers: the LDS reads for code
// dword d+1 are issued before the adds of dword d, so each add consumes a
// value read one dword earlier and LDS latency overlaps the add chain.
template <int KIND, int GROUP>
__device__ __forceinline__ void compute_window(const WindowState<KIND, GROUP> &st, const float *T, float &sum,
                                               float &gd, int w, int groups, int windows_per_group) {
    using S = TableShape<KIND>;
    constexpr int NN = WindowState<KIND, GROUP>::kNorms;
    constexpr int D = S::kChunksPerWindow * 4;  // code dwords per window
    const int gbase = w * NN;                   // first group index closing in this window (GROUP > 0)
    constexpr int P = ND_PIPE;  // code dwords read ahead of the adds
    SlotValues<KIND> v[P + 1];
#pragma unroll
    for (int dn = 0; dn < P && dn < D; ++dn) {
        const u32x4 &cn = st.codes[dn >> 2];
        const uint32_t wn = (dn & 3) == 0 ? cn.x : (dn & 3) == 1 ? cn.y : (dn & 3) == 2 ? cn.z : cn.w;
        uint32_t off[8];
        slot_offsets<KIND>(wn, off);
        read_slots<KIND>(T, dn * 8, off, v[dn % (P + 1)]);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (d + P < D) {
            const int dn = d + P;
            const u32x4 &cn = st.codes[dn >> 2];
            const uint32_t wn = (dn & 3) == 0 ? cn.x : (dn & 3) == 1 ? cn.y : (dn & 3) == 2 ? cn.z : cn.w;
            uint32_t off[8];
            slot_offsets<KIND>(wn, off);
            read_slots<KIND>(T, dn * 8, off, v[dn % (P + 1)]);
        }
        // compiler-only fence: keeps each dword's LDS reads in its pipeline
        // slot (otherwise every read of the window is hoisted and spilled)
        asm volatile("" ::: "memory");
        if (ND_SCHED_BARRIER) __builtin_amdgcn_sched_barrier(0);
        const SlotValues<KIND> &cur = v[d % (P + 1)];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            gd += cur.a[i];
            if constexpr (KIND == kCrumb) gd += cur.b[i];
            if constexpr (GROUP > 0) {
                const int pos_end = (d * 8 + i + 1) * S::kPositionsPerSlot;  // positions consumed in window
                if (pos_end % GROUP == 0) {
                    const int k = pos_end / GROUP - 1;
                    if (gbase + k < groups) sum += gd * h2f(st.norms[k]);
                    gd = 0.0f;
                }
            }
        }
        // pins this dword's adds before the next dword's reads (the fence
        // above only orders memory operations)
        asm volatile("" : "+v"(gd), "+v"(sum));
        if (ND_SCHED_BARRIER) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (GROUP == 0) {
        if ((w + 1) % windows_per_group == 0) {
            if (w / windows_per_group < groups) sum += gd * h2f(st.norms[0]);
            gd = 0.0f;
        }
    }
}

template <int KIND, int GROUP>
__global__ __launch_bounds__(kRowsPerBlock, 2) void cq_gemv_kernel(CqJob job0, const CqJob *__restrict__ jobs, int njobs,
                                                                CqGeom geom) {
    using S = TableShape<KIND>;
    __shared__ __attribute__((aligned(16))) float T[2][S::kFloats];
    __shared__ float stage[GROUP > 64 ? kWindow : 1];
    constexpr int PPT = kPositionsPerThread;

    const int blk = blockIdx.x;
    CqJob J = job0;
    if (njobs > 0) {
        const ND_CONST CqJob *cj = (const ND_CONST CqJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J.codes = cj[j].codes;
        J.norms = cj[j].norms;
        J.act = cj[j].act;
        J.y = cj[j].y;
        J.rows = cj[j].rows;
        J.n_pad = cj[j].n_pad;
        J.block_begin = cj[j].block_begin;
        J.batch = cj[j].batch;
    }
    const int rows = J.rows, batch = J.batch;
    const int tile = blk - J.block_begin;
    const int row = tile * kRowsPerBlock + threadIdx.x;
    // this workgroup's row tile of codes and norms
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms =
        buffer_rsrc(J.norms + static_cast<size_t>(tile) * geom.groups * kRowsPerBlock,
                    static_cast<uint32_t>(geom.groups) * kRowsPerBlock * 2u);
    const int windows = geom.windows, groups = geom.groups, in = geom.in;
    const int wpg = GROUP == 0 ? geom.group / kWindow : 1;
    const int act_stride = GROUP > 0 ? in : windows * kWindow;
    const float scale = geom.scale;
    float lut[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) lut[i] = geom.lut[i];

    for (int b = 0; b < batch; ++b) {
        const __amdgpu_buffer_rsrc_t act =
            buffer_rsrc(J.act + static_cast<size_t>(b) * act_stride, static_cast<uint32_t>(act_stride) * 4u);
        WindowState<KIND, GROUP> cur, nxt;
        float xa[PPT];
        load_act(act, 0, xa);
        load_window<KIND, GROUP>(cur, codes, norms, 0, groups, wpg);
        __syncthreads();  // the previous batch row finished reading T[0]
        if constexpr (GROUP > 0) window_fwht<GROUP>(xa, scale, stage);
        build_table<KIND>(T[0], lut, xa);
        __syncthreads();
        float sum = 0.0f, gd = 0.0f;
        // Two windows per iteration so each table buffer index is a constant.
        // Per window: issue the next window's activation and code loads (in that
        // order, unconditionally, clamped at the last window), sum this window
        // from its table, then transform the next activations and build the
        // next table in the other buffer; one barrier per window. Every loaded
        // value is consumed within the iteration that loads it, so no register
        // copy of a pending load (and no full vector-memory wait) is needed.
        for (int w = 0; w < windows; w += 2) {
            const int w1 = min(w + 1, windows - 1);
            load_act(act, w1, xa);
            load_window<KIND, GROUP>(nxt, codes, norms, w1, groups, wpg);
            compute_window<KIND, GROUP>(cur, T[0], sum, gd, w, groups, wpg);
            if (w + 1 < windows) {
                if constexpr (GROUP > 0) window_fwht<GROUP>(xa, scale, stage);
                build_table<KIND>(T[1], lut, xa);
            }
            __syncthreads();
            if (w + 1 >= windows) break;
            const int w2 = min(w + 2, windows - 1);
            load_act(act, w2, xa);
            load_window<KIND, GROUP>(cur, codes, norms, w2, groups, wpg);
            compute_window<KIND, GROUP>(nxt, T[1], sum, gd, w + 1, groups, wpg);
            if (w + 2 < windows) {
                if constexpr (GROUP > 0) window_fwht<GROUP>(xa, scale, stage);
                build_table<KIND>(T[0], lut, xa);
            }
            __syncthreads();
        }
        if (row < rows) ((ND_GLOBAL float *)J.y)[static_cast<size_t>(b) * rows + row] = sum;
    }
}

// ---------------------------------------------------------------------------
// Split-window FP32 GEMV (groups of 8 .. 128 positions)
//
// Two threads per output row: a workgroup of 512 threads covers a 256-row
// tile, and its two halves (waves 0-3 and 4-7) take the lower and upper half
// of every window's groups against one shared product table. Per-group
// results p_g = gd_g * half(norm_g) are independent, so each half computes
// its own groups with the reference's sequential code order; the lower half
// owns the row sum and adds the upper half's p_g (handed over through LDS,
// double-buffered by window parity) right after its own, so the row sum still
// runs over g = 0, 1, 2, ... exactly as cq.cpp:157-164 does: bit-identical.
// This doubles the waves in flight (4 per SIMD) and halves the code registers
// each lane holds in its prefetch.
//
// Code extraction: the table entry of a 4-bit code is code*4 bytes into its
// slot (code*8 for a 2-bit pair). With the code dword rotated left by 2 (3),
// every even nibble sits at bits 2-5 (3-6) of a byte, and rotated right by 2
// (1), every odd one does; one SDWA `and` with a byte select then yields a
// slot offset, so a code costs one VALU op, one LDS read and one add.
// ---------------------------------------------------------------------------
constexpr int kSplitThreads = 2 * kRowsPerBlock;

template <int KIND, int GROUP>
struct SplitShape {
    static constexpr int kChunks = TableShape<KIND>::kChunksPerWindow / 2;  // chunks per half window
    static constexpr int kDwords = kChunks * 4;
    static constexpr int kSlotsPerHalf = TableShape<KIND>::kSlots / 2;
    static constexpr int kGroupsPerHalf = kWindow / GROUP / 2;
    static_assert(GROUP >= 8 && GROUP <= kWindow / 2, "split GEMV takes groups of at most half a window");
};

template <int KIND, int GROUP>
struct HalfState {
    u32x4 codes[SplitShape<KIND, GROUP>::kChunks];
    uint16_t norms[SplitShape<KIND, GROUP>::kGroupsPerHalf];
};

// (x byte BYTE) & mask, one SDWA op; mask lives in an SGPR.
template <int BYTE>
__device__ __forceinline__ uint32_t and_byte(uint32_t mask, uint32_t x) {
    uint32_t r;
    if constexpr (BYTE == 0)
        asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
            : "=v"(r) : "s"(mask), "v"(x));
    else if constexpr (BYTE == 1)
        asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
            : "=v"(r) : "s"(mask), "v"(x));
    else if constexpr (BYTE == 2)
        asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
            : "=v"(r) : "s"(mask), "v"(x));
    else
        asm("v_and_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
            : "=v"(r) : "s"(mask), "v"(x));
    return r;
}

// Byte offsets of the 8 table entries addressed by one code dword, in code
// order: off[2m] from nibble 2m, off[2m+1] from nibble 2m+1.
template <int KIND>
__device__ __forceinline__ void slot_offsets_sdwa(uint32_t wd, uint32_t mask, uint32_t off[8]) {
    constexpr int kRot = KIND == kNib ? 2 : 3;                      // log2(entry bytes)
    const uint32_t X = __builtin_amdgcn_alignbit(wd, wd, 32 - kRot);  // rotate left: even nibbles
    const uint32_t Y = __builtin_amdgcn_alignbit(wd, wd, 4 - kRot);   // rotate right: odd nibbles
    off[0] = and_byte<0>(mask, X);
    off[1] = and_byte<0>(mask, Y);
    off[2] = and_byte<1>(mask, X);
    off[3] = and_byte<1>(mask, Y);
    off[4] = and_byte<2>(mask, X);
    off[5] = and_byte<2>(mask, Y);
    off[6] = and_byte<3>(mask, X);
    off[7] = and_byte<3>(mask, Y);
}

// Byte offset of window w's activations (wave-uniform, kept scalar).
__device__ __forceinline__ int window_offset(int w) { return __builtin_amdgcn_readfirstlane(w * kWindow * 4); }

// Loads of this thread's half of window w: code chunk c (of the half's
// kChunks) and the norm of the half's group k. Both buffer resources end at
// the tile's last window / group, so windows past the end read zero without
// touching memory (the rolling prefetch below runs two windows ahead
// unconditionally; phantom groups never reach the row sum).
template <int KIND, int GROUP>
__device__ __forceinline__ u32x4 load_chunk(__amdgpu_buffer_rsrc_t codes, int w, int half, int r, int c) {
    using H = SplitShape<KIND, GROUP>;
    constexpr int C = TableShape<KIND>::kChunksPerWindow;
    const int soff = __builtin_amdgcn_readfirstlane((w * C + half * H::kChunks + c) * kRowsPerBlock * 16);
    return __builtin_amdgcn_raw_buffer_load_b128(codes, r * 16u, soff, 0);
}

template <int KIND, int GROUP>
__device__ __forceinline__ uint16_t load_norm(__amdgpu_buffer_rsrc_t norms, int w, int half, int r, int k) {
    using H = SplitShape<KIND, GROUP>;
    const int g = w * (2 * H::kGroupsPerHalf) + half * H::kGroupsPerHalf + k;
    return __builtin_amdgcn_raw_buffer_load_b16(norms, r * 2u, __builtin_amdgcn_readfirstlane(g * kRowsPerBlock * 2),
                                                0);
}

template <int KIND, int GROUP>
__device__ __forceinline__ void load_half(HalfState<KIND, GROUP> &st, __amdgpu_buffer_rsrc_t codes,
                                          __amdgpu_buffer_rsrc_t norms, int w, int half, int r) {
    using H = SplitShape<KIND, GROUP>;
#pragma unroll
    for (int c = 0; c < H::kChunks; ++c) st.codes[c] = load_chunk<KIND, GROUP>(codes, w, half, r, c);
#pragma unroll
    for (int k = 0; k < H::kGroupsPerHalf; ++k) st.norms[k] = load_norm<KIND, GROUP>(norms, w, half, r, k);
}

// One half window in the reference's order. Without PARK (the lower half)
// each closed group is added into the row sum; with PARK (by default the
// upper half) p_g goes to P[k][r] for the row sum's owner.
template <int KIND, int GROUP, int HALF, bool PARK = HALF == 1>
__device__ __forceinline__ void compute_half(HalfState<KIND, GROUP> &st, const float *T, float *P, int r,
                                             uint32_t mask, float &sum, float &gd, int w, int groups,
                                             __amdgpu_buffer_rsrc_t codes, __amdgpu_buffer_rsrc_t norms) {
    using S = TableShape<KIND>;
    using H = SplitShape<KIND, GROUP>;
    constexpr int D = H::kDwords;
    constexpr int P_AHEAD = ND_PIPE;
    const int gbase = w * (2 * H::kGroupsPerHalf) + HALF * H::kGroupsPerHalf;  // first group of this half
    SlotValues<KIND> v[P_AHEAD + 1];
#pragma unroll
    for (int dn = 0; dn < P_AHEAD && dn < D; ++dn) {
        const u32x4 &cn = st.codes[dn >> 2];
        const uint32_t wn = (dn & 3) == 0 ? cn.x : (dn & 3) == 1 ? cn.y : (dn & 3) == 2 ? cn.z : cn.w;
        uint32_t off[8];
        slot_offsets_sdwa<KIND>(wn, mask, off);
        read_slots<KIND>(T, HALF * H::kSlotsPerHalf + dn * 8, off, v[dn % (P_AHEAD + 1)]);
        if ((dn & 3) == 3) st.codes[dn >> 2] = load_chunk<KIND, GROUP>(codes, w + 2, HALF, r, dn >> 2);
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (d + P_AHEAD < D) {
            const int dn = d + P_AHEAD;
            const u32x4 &cn = st.codes[dn >> 2];
            const uint32_t wn = (dn & 3) == 0 ? cn.x : (dn & 3) == 1 ? cn.y : (dn & 3) == 2 ? cn.z : cn.w;
            uint32_t off[8];
            slot_offsets_sdwa<KIND>(wn, mask, off);
            read_slots<KIND>(T, HALF * H::kSlotsPerHalf + dn * 8, off, v[dn % (P_AHEAD + 1)]);
            // chunk dn / 4 is spent: refill it with the same chunk two windows ahead
            if ((dn & 3) == 3) st.codes[dn >> 2] = load_chunk<KIND, GROUP>(codes, w + 2, HALF, r, dn >> 2);
        }
        asm volatile("" ::: "memory");
        if (ND_SCHED_BARRIER) __builtin_amdgcn_sched_barrier(0);
        const SlotValues<KIND> &cur = v[d % (P_AHEAD + 1)];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            gd += cur.a[i];
            if constexpr (KIND == kCrumb) gd += cur.b[i];
            const int pos_end = (d * 8 + i + 1) * S::kPositionsPerSlot;  // positions consumed in this half
            if (pos_end % GROUP == 0) {
                const int k = pos_end / GROUP - 1;
                const float p = gd * h2f(st.norms[k]);
                if constexpr (!PARK) {
                    if (gbase + k < groups) sum += p;
                } else {
                    P[k * kRowsPerBlock + r] = p;
                }
                gd = 0.0f;
                st.norms[k] = load_norm<KIND, GROUP>(norms, w + 2, HALF, r, k);
            }
        }
        asm volatile("" : "+v"(gd), "+v"(sum));
        if (ND_SCHED_BARRIER) __builtin_amdgcn_sched_barrier(0);
    }
}

// Lower half: add the upper half's p_g of window w (parked in P) in group order.
template <int KIND, int GROUP>
__device__ __forceinline__ void add_upper(const float *P, int r, float &sum, int w, int groups) {
    using H = SplitShape<KIND, GROUP>;
    const int gbase = w * (2 * H::kGroupsPerHalf) + H::kGroupsPerHalf;
#pragma unroll
    for (int k = 0; k < H::kGroupsPerHalf; ++k)
        if (gbase + k < groups) sum += P[k * kRowsPerBlock + r];
}

// Table build for the split kernel: thread (half, r) owns window position r
// and writes half of that position's entries (4-bit: codes 8*half .. +7;
// 2-bit: pair entries with high code 2*half, 2*half+1).
template <int KIND>
__device__ __forceinline__ void build_table_half(float *__restrict__ T, const float *lut, float x, int half, int r) {
    using S = TableShape<KIND>;
    if constexpr (KIND == kNib) {
        float *dst = T + r * S::kSlotFloats + half * 8;
#pragma unroll
        for (int c = 0; c < 8; ++c) dst[c] = lut[half * 8 + c] * x;
    } else {
        const int lane = r & 63;
        const int l = lane & 31;
        const float r0 = __shfl(x, 2 * l);
        const float r1 = __shfl(x, 2 * l + 1);
        if (lane < 32) {
            float p0[4], p1[2];
#pragma unroll
            for (int c = 0; c < 4; ++c) p0[c] = lut[c] * r0;
#pragma unroll
            for (int c = 0; c < 2; ++c) p1[c] = lut[half * 2 + c] * r1;
            const int slot = (r & ~63) / 2 + l;
            float4 *dst = reinterpret_cast<float4 *>(T + slot * S::kSlotFloats);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int hi = half * 2 + c;
                dst[2 * hi] = make_float4(p0[0], p1[c], p0[1], p1[c]);
                dst[2 * hi + 1] = make_float4(p0[2], p1[c], p0[3], p1[c]);
            }
        }
    }
}

// All batch rows of one row tile for one half of the split kernel.
template <int KIND, int GROUP, int HALF>
__device__ __forceinline__ void split_rows(const CqJob &J, const CqGeom &geom, float (*T)[TableShape<KIND>::kFloats],
                                           float (*P)[SplitShape<KIND, GROUP>::kGroupsPerHalf * kRowsPerBlock],
                                           float *stage, int blk) {
    const int r = threadIdx.x % kRowsPerBlock;
    const int rows = J.rows, batch = J.batch;
    const int tile = blk - J.block_begin;
    const int row = tile * kRowsPerBlock + r;
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms =
        buffer_rsrc(J.norms + static_cast<size_t>(tile) * geom.groups * kRowsPerBlock,
                    static_cast<uint32_t>(geom.groups) * kRowsPerBlock * 2u);
    const int windows = geom.windows, groups = geom.groups, in = geom.in;
    const float scale = geom.scale;
    const uint32_t mask = KIND == kNib ? 0x3Cu : 0x78u;
    float lut[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) lut[i] = geom.lut[i];

    for (int b = 0; b < batch; ++b) {
        const __amdgpu_buffer_rsrc_t act =
            buffer_rsrc(J.act + static_cast<size_t>(b) * in, static_cast<uint32_t>(in) * 4u);
        HalfState<KIND, GROUP> cur, nxt;
        float xa[1];
        xa[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(act, r * 4u, 0, 0));
        load_half<KIND, GROUP>(cur, codes, norms, 0, HALF, r);
        load_half<KIND, GROUP>(nxt, codes, norms, 1, HALF, r);
        __syncthreads();  // the previous batch row finished with T[0] and P
        window_fwht<GROUP>(xa, scale, stage);
        build_table_half<KIND>(T[0], lut, xa[0], HALF, r);
        xa[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(act, r * 4u, kWindow * 4, 0));
        __syncthreads();
        float sum = 0.0f, gd = 0.0f;
        // Whole window pairs, then the last window if the count is odd; one
        // barrier per window and no condition around any load, so every
        // iteration issues the same loads in the same order. Window w is
        // summed from `cur` (even) or `nxt` (odd), whose chunks are refilled
        // with window w + 2 as they are spent: loads stream continuously two
        // windows ahead. The activations of window w + 1 (loaded one window
        // earlier) then become its table (a window past the end reads zeros
        // into a buffer nobody reads again) and those of window w + 2 are
        // requested. Before its own groups of window w the lower half adds the
        // upper half's groups of window w - 1 (P[(w - 1) & 1]).
        const int pairs = windows / 2;
        for (int it = 0; it < pairs; ++it) {
            const int w = 2 * it;
            if (HALF == 0 && it > 0) add_upper<KIND, GROUP>(P[1], r, sum, w - 1, groups);
            compute_half<KIND, GROUP, HALF>(cur, T[0], P[0], r, mask, sum, gd, w, groups, codes, norms);
            window_fwht<GROUP>(xa, scale, stage);
            build_table_half<KIND>(T[1], lut, xa[0], HALF, r);
            xa[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(act, r * 4u, window_offset(w + 2), 0));
            __syncthreads();
            if (HALF == 0) add_upper<KIND, GROUP>(P[0], r, sum, w, groups);
            compute_half<KIND, GROUP, HALF>(nxt, T[1], P[1], r, mask, sum, gd, w + 1, groups, codes, norms);
            window_fwht<GROUP>(xa, scale, stage);
            build_table_half<KIND>(T[0], lut, xa[0], HALF, r);
            xa[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(act, r * 4u, window_offset(w + 3), 0));
            __syncthreads();
        }
        if (windows & 1) {
            const int w = windows - 1;
            if (HALF == 0 && w > 0) add_upper<KIND, GROUP>(P[1], r, sum, w - 1, groups);
            compute_half<KIND, GROUP, HALF>(cur, T[0], P[0], r, mask, sum, gd, w, groups, codes, norms);
            __syncthreads();
        }
        if (HALF == 0) {
            add_upper<KIND, GROUP>(P[(windows - 1) & 1], r, sum, windows - 1, groups);
            if (row < rows) ((ND_GLOBAL float *)J.y)[static_cast<size_t>(b) * rows + row] = sum;
        }
    }
}

template <int KIND, int GROUP>
__global__ __launch_bounds__(kSplitThreads, 4) void cq_gemv_split_kernel(CqJob job0, const CqJob *__restrict__ jobs,
                                                                       int njobs, CqGeom geom) {
    using S = TableShape<KIND>;
    using H = SplitShape<KIND, GROUP>;
    __shared__ __attribute__((aligned(16))) float T[2][S::kFloats];
    __shared__ float P[2][H::kGroupsPerHalf * kRowsPerBlock];
    __shared__ float stage[GROUP > 64 ? 2 * kWindow : 1];
    static_assert(kPositionsPerThread == 1, "split GEMV assumes one window position per row thread");

    const int blk = blockIdx.x;
    CqJob J = job0;
    if (njobs > 0) {
        const ND_CONST CqJob *cj = (const ND_CONST CqJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J.codes = cj[j].codes;
        J.norms = cj[j].norms;
        J.act = cj[j].act;
        J.y = cj[j].y;
        J.rows = cj[j].rows;
        J.n_pad = cj[j].n_pad;
        J.block_begin = cj[j].block_begin;
        J.batch = cj[j].batch;
    }
    // The half is a compile-time constant of each copy of the window loop, so
    // each copy is straight-line code whose load/wait bookkeeping does not mix
    // with the other half's.
    if (__builtin_amdgcn_readfirstlane(threadIdx.x / kRowsPerBlock) == 0)
        split_rows<KIND, GROUP, 0>(J, geom, T, P, stage, blk);
    else
        split_rows<KIND, GROUP, 1>(J, geom, T, P, stage, blk);
}

// ---------------------------------------------------------------------------
// Window-parallel split GEMV for inputs of two windows (257 .. 512 positions,
// groups of 128: a decode step's attention projections)
//
// Four threads per output row: part q = (window q / 2, half q % 2) builds its
// half of window q / 2's table (each window has its own) and runs that half
// with the split kernel's code, so the two windows are computed at once
// instead of in turn. Window 0's lower half owns the row sum: after its own
// groups it adds the parked p_g of window 0's upper half, then of window 1's
// lower and upper halves, i.e. g = 0, 1, 2, ... as cq.cpp:157-164 sums:
// bit-identical with the split kernel.
// ---------------------------------------------------------------------------
constexpr int kWsplitThreads = 4 * kRowsPerBlock;

template <int KIND, int GROUP, int PART>
__device__ __forceinline__ void wsplit_rows(const CqJob &J, const CqGeom &geom,
                                            float (*T)[TableShape<KIND>::kFloats],
                                            float (*P)[SplitShape<KIND, GROUP>::kGroupsPerHalf * kRowsPerBlock],
                                            float *stage, int blk) {
    using H = SplitShape<KIND, GROUP>;
    constexpr int WW = PART / 2, HALF = PART % 2;
    const int r = threadIdx.x % kRowsPerBlock;
    const int rows = J.rows, batch = J.batch;
    const int tile = blk - J.block_begin;
    const int row = tile * kRowsPerBlock + r;
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms =
        buffer_rsrc(J.norms + static_cast<size_t>(tile) * geom.groups * kRowsPerBlock,
                    static_cast<uint32_t>(geom.groups) * kRowsPerBlock * 2u);
    const int groups = geom.groups, in = geom.in;
    const float scale = geom.scale;
    const uint32_t mask = KIND == kNib ? 0x3Cu : 0x78u;
    float lut[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) lut[i] = geom.lut[i];

    for (int b = 0; b < batch; ++b) {
        const __amdgpu_buffer_rsrc_t act =
            buffer_rsrc(J.act + static_cast<size_t>(b) * in, static_cast<uint32_t>(in) * 4u);
        HalfState<KIND, GROUP> cur;
        float xa[1];
        xa[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(act, r * 4u, window_offset(WW), 0));
        load_half<KIND, GROUP>(cur, codes, norms, WW, HALF, r);
        __syncthreads();  // the previous batch row finished with T and P
        window_fwht<GROUP>(xa, scale, stage);
        build_table_half<KIND>(T[WW], lut, xa[0], HALF, r);
        __syncthreads();
        float sum = 0.0f, gd = 0.0f;
        compute_half<KIND, GROUP, HALF, PART != 0>(cur, T[WW], P[PART == 0 ? 0 : PART - 1], r, mask, sum, gd, WW,
                                                   groups, codes, norms);
        __syncthreads();
        if constexpr (PART == 0) {
#pragma unroll
            for (int q = 0; q < 3; ++q) {  // parts 1, 2, 3: groups after window 0's lower half, in order
                const int gbase = (q + 1) * H::kGroupsPerHalf;
#pragma unroll
                for (int k = 0; k < H::kGroupsPerHalf; ++k)
                    if (gbase + k < groups) sum += P[q][k * kRowsPerBlock + r];
            }
            if (row < rows) ((ND_GLOBAL float *)J.y)[static_cast<size_t>(b) * rows + row] = sum;
        }
    }
}

template <int KIND, int GROUP>
__global__ __launch_bounds__(kWsplitThreads) void cq_gemv_wsplit_kernel(CqJob job0, const CqJob *__restrict__ jobs,
                                                                       int njobs, CqGeom geom) {
    using S = TableShape<KIND>;
    using H = SplitShape<KIND, GROUP>;
    __shared__ __attribute__((aligned(16))) float T[2][S::kFloats];
    __shared__ float P[3][H::kGroupsPerHalf * kRowsPerBlock];
    __shared__ float stage[GROUP > 64 ? 4 * kWindow : 1];
    static_assert(kPositionsPerThread == 1, "window-parallel GEMV assumes one window position per row thread");

    const int blk = blockIdx.x;
    CqJob J = job0;
    if (njobs > 0) {
        const ND_CONST CqJob *cj = (const ND_CONST CqJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J.codes = cj[j].codes;
        J.norms = cj[j].norms;
        J.act = cj[j].act;
        J.y = cj[j].y;
        J.rows = cj[j].rows;
        J.n_pad = cj[j].n_pad;
        J.block_begin = cj[j].block_begin;
        J.batch = cj[j].batch;
    }
    switch (__builtin_amdgcn_readfirstlane(threadIdx.x / kRowsPerBlock)) {
    case 0: wsplit_rows<KIND, GROUP, 0>(J, geom, T, P, stage, blk); break;
    case 1: wsplit_rows<KIND, GROUP, 1>(J, geom, T, P, stage, blk); break;
    case 2: wsplit_rows<KIND, GROUP, 2>(J, geom, T, P, stage, blk); break;
    default: wsplit_rows<KIND, GROUP, 3>(J, geom, T, P, stage, blk); break;
    }
}

// Inputs of two windows with groups of 128 take the window-parallel kernel
// (NEEDLE2_GPU_FP32_WSPLIT=never: the split kernel).
static bool wsplit_wanted(const CqGeom &g) {
    const char *mode = std::getenv("NEEDLE2_GPU_FP32_WSPLIT");
    return g.windows == 2 && g.group == 128 && !(mode && std::strcmp(mode, "never") == 0);
}

// ---------------------------------------------------------------------------
// Quarter-split FP32 GEMV (groups of 8 .. 64 positions)
//
// Four threads per output row: a 1024-thread workgroup covers a 256-row tile
// and its quarters (waves 0-3, 4-7, 8-11, 12-15) take positions
// [64q, 64q + 64) of every 256-position window against one shared product
// table. As in the split kernel, each quarter computes its own groups in the
// reference's code order, quarters 1-3 park their p_g in LDS and quarter 0
// adds them right after its own, in group order: bit-identical to
// cq.cpp:157-164. With 64 codes per thread per window the registers fit 64
// VGPRs, so two workgroups give 8 waves per SIMD, which the LDS lookups need
// to run near the LDS read rate.
//
// The activations arrive already transformed (rot = per-group FWHT of x,
// zero past the padded length; one pre-pass launch for all inputs), so a
// thread's per-window table work is one activation load, four products and
// one 16-byte LDS store: slot p holds cb[c] * rot[p] for the 16 codes c at a
// 20-float stride (conflict-free for both the 16-byte stores and the
// per-code 4-byte reads); 2-bit slots hold (cb[c0] * rot[2s], cb[c1] * rot[2s+1])
// pairs at a 36-float stride.
// ---------------------------------------------------------------------------
constexpr int kQuads = 4;
constexpr int kQuadThreads = kQuads * kRowsPerBlock;

template <int KIND, int GROUP>
struct QuadShape {
    static constexpr int kPositions = kWindow / kQuads;                          // per quarter window
    static constexpr int kChunks = kPositions / TableShape<KIND>::kCodesPerChunk;  // 2 (4-bit) or 1 (2-bit)
    static constexpr int kDwords = kChunks * 4;
    static constexpr int kSlots = kPositions / TableShape<KIND>::kPositionsPerSlot;
    static constexpr int kGroups = kPositions / GROUP;                           // groups per quarter window
    static constexpr int kSlotFloats = KIND == kNib ? 20 : 36;
    static constexpr int kFloats = (kWindow / TableShape<KIND>::kPositionsPerSlot) * kSlotFloats;
    static constexpr int kPipe = KIND == kNib && GROUP >= 32 ? 2 : 1;             // code dwords read ahead
    static_assert(GROUP >= 8 && GROUP <= kPositions, "quarter GEMV takes groups of at most 64 positions");
};

template <int KIND, int GROUP>
struct QuadState {
    u32x4 codes[QuadShape<KIND, GROUP>::kChunks];
    uint16_t norms[QuadShape<KIND, GROUP>::kGroups];
};

template <int KIND, int GROUP>
__device__ __forceinline__ u32x4 quad_chunk(__amdgpu_buffer_rsrc_t codes, int w, int q, int r, int c) {
    constexpr int C = TableShape<KIND>::kChunksPerWindow;
    const int soff =
        __builtin_amdgcn_readfirstlane((w * C + q * QuadShape<KIND, GROUP>::kChunks + c) * kRowsPerBlock * 16);
    return __builtin_amdgcn_raw_buffer_load_b128(codes, r * 16u, soff, kStreamLoad);
}

template <int KIND, int GROUP>
__device__ __forceinline__ uint16_t quad_norm(__amdgpu_buffer_rsrc_t norms, int w, int q, int r, int k) {
    constexpr int NQ = QuadShape<KIND, GROUP>::kGroups;
    const int g = w * (kQuads * NQ) + q * NQ + k;
    return __builtin_amdgcn_raw_buffer_load_b16(norms, r * 2u, __builtin_amdgcn_readfirstlane(g * kRowsPerBlock * 2),
                                                0);
}

template <int KIND, int GROUP>
__device__ __forceinline__ void quad_load(QuadState<KIND, GROUP> &st, __amdgpu_buffer_rsrc_t codes,
                                          __amdgpu_buffer_rsrc_t norms, int w, int q, int r) {
    using Q = QuadShape<KIND, GROUP>;
#pragma unroll
    for (int c = 0; c < Q::kChunks; ++c) st.codes[c] = quad_chunk<KIND, GROUP>(codes, w, q, r, c);
#pragma unroll
    for (int k = 0; k < Q::kGroups; ++k) st.norms[k] = quad_norm<KIND, GROUP>(norms, w, q, r, k);
}

// Transformed activations this thread turns into table entries: position r
// (4-bit) or positions 2(r/2), 2(r/2)+1 (2-bit) of window w; past the end: 0.
template <int KIND>
__device__ __forceinline__ float2 quad_act(__amdgpu_buffer_rsrc_t rot, int w, int r) {
    if constexpr (KIND == kNib) {
        return make_float2(
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rot, r * 4u, window_offset(w), 0)), 0.0f);
    } else {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rot, (r >> 1) * 8u, window_offset(w), 0);
        return __builtin_bit_cast(float2, v);
    }
}

// The same values from the raw input row (XF): the thread loads its position(s)
// of window w (zeros past the row, the reference's padding) and runs the group
// FWHT as rot_many_kernel does: the stages in ascending order with the
// reference's operands, each stride h < 64 between lanes (2-bit: stride 1
// inside the lane, which holds positions 2m and 2m + 1, and stride h >= 2 with
// lane l ^ h, since lanes 2m and 2m + 1 hold the same pair), then * scale.
template <int KIND, int GROUP>
__device__ __forceinline__ float2 quad_act_x(__amdgpu_buffer_rsrc_t x, int w, int r, float scale) {
    const int lane = r & 63;
    if constexpr (KIND == kNib) {
        float v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x, r * 4u, window_offset(w), 0));
        wave_butterflies<GROUP, 1>(v, lane);
        return make_float2(v * scale, 0.0f);
    } else {
        const float x0 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x, (r >> 1) * 8u, window_offset(w), 0));
        const float x1 =
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x, (r >> 1) * 8u + 4u, window_offset(w), 0));
        float a = x0 + x1, b = x0 - x1;
        wave_butterflies<GROUP, 2>(a, lane);
        wave_butterflies<GROUP, 2>(b, lane);
        return make_float2(a * scale, b * scale);
    }
}

// Quarter q's share of the table of one window: 4-bit slot r, codes 4q..4q+3;
// 2-bit slot r/2, pair entries c0 | q << 2 for c0 = 2(r&1), 2(r&1)+1.
template <int KIND, int GROUP>
__device__ __forceinline__ void quad_build(float *__restrict__ T, const float *lut, float2 x, int q, int r) {
    using Q = QuadShape<KIND, GROUP>;
    if constexpr (KIND == kNib) {
        *reinterpret_cast<float4 *>(T + r * Q::kSlotFloats + 4 * q) =
            make_float4(lut[4 * q] * x.x, lut[4 * q + 1] * x.x, lut[4 * q + 2] * x.x, lut[4 * q + 3] * x.x);
    } else {
        const int part = r & 1;
        const float hi = lut[q] * x.y;
        *reinterpret_cast<float4 *>(T + (r >> 1) * Q::kSlotFloats + 8 * q + 4 * part) =
            make_float4(lut[2 * part] * x.x, hi, lut[2 * part + 1] * x.x, hi);
    }
}

// One quarter window in the reference's order, refilling each spent chunk /
// norm with window w + 2 (REFILL; a pass over the same codes for another
// activation row keeps them). Quarter 0 adds closed groups into the row sum;
// quarters 1-3 park p_g in P[q - 1][k][r].
template <int KIND, int GROUP, int QUAD, bool REFILL = true>
__device__ __forceinline__ void quad_compute(QuadState<KIND, GROUP> &st, const float *T, float *P, int r,
                                             uint32_t mask, float &sum, float &gd, int w, int groups,
                                             __amdgpu_buffer_rsrc_t codes, __amdgpu_buffer_rsrc_t norms) {
    using S = TableShape<KIND>;
    using Q = QuadShape<KIND, GROUP>;
    constexpr int D = Q::kDwords;
    constexpr int PA = Q::kPipe;
    const int gbase = w * (kQuads * Q::kGroups);  // quarter 0's first group
    SlotValues<KIND> v[PA + 1];
    auto issue = [&](int dn) {
        const u32x4 &cn = st.codes[dn >> 2];
        const uint32_t wn = (dn & 3) == 0 ? cn.x : (dn & 3) == 1 ? cn.y : (dn & 3) == 2 ? cn.z : cn.w;
        uint32_t off[8];
        slot_offsets_sdwa<KIND>(wn, mask, off);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const char *slot = reinterpret_cast<const char *>(T + (QUAD * Q::kSlots + dn * 8 + i) * Q::kSlotFloats);
            if constexpr (KIND == kNib) {
                v[dn % (PA + 1)].a[i] = *reinterpret_cast<const float *>(slot + off[i]);
            } else {
                const float2 pr = *reinterpret_cast<const float2 *>(slot + off[i]);
                v[dn % (PA + 1)].a[i] = pr.x;
                v[dn % (PA + 1)].b[i] = pr.y;
            }
        }
        if (REFILL && (dn & 3) == 3) st.codes[dn >> 2] = quad_chunk<KIND, GROUP>(codes, w + 2, QUAD, r, dn >> 2);
    };
#pragma unroll
    for (int dn = 0; dn < PA && dn < D; ++dn) issue(dn);
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (d + PA < D) issue(d + PA);
        asm volatile("" ::: "memory");
        if (ND_SCHED_BARRIER) __builtin_amdgcn_sched_barrier(0);
        const SlotValues<KIND> &cur = v[d % (PA + 1)];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            gd += cur.a[i];
            if constexpr (KIND == kCrumb) gd += cur.b[i];
            const int pos_end = (d * 8 + i + 1) * S::kPositionsPerSlot;  // positions consumed in this quarter
            if (pos_end % GROUP == 0) {
                const int k = pos_end / GROUP - 1;
                const float p = gd * h2f(st.norms[k]);
                if constexpr (QUAD == 0) {
                    if (gbase + k < groups) sum += p;
                } else {
                    P[((QUAD - 1) * Q::kGroups + k) * kRowsPerBlock + r] = p;
                }
                gd = 0.0f;
                if (REFILL) st.norms[k] = quad_norm<KIND, GROUP>(norms, w + 2, QUAD, r, k);
            }
        }
        asm volatile("" : "+v"(gd), "+v"(sum));
        if (ND_SCHED_BARRIER) __builtin_amdgcn_sched_barrier(0);
    }
}

// Quarter 0: add quarters 1-3's p_g of window w (parked in P) in group order.
template <int KIND, int GROUP>
__device__ __forceinline__ void quad_add_parked(const float *P, int r, float &sum, int w, int groups) {
    using Q = QuadShape<KIND, GROUP>;
    const int gbase = w * (kQuads * Q::kGroups) + Q::kGroups;
#pragma unroll
    for (int k = 0; k < (kQuads - 1) * Q::kGroups; ++k)
        if (gbase + k < groups) sum += P[k * kRowsPerBlock + r];
}

// XF: J.act is the raw input ([batch][in]), transformed here (quad_act_x),
// instead of the pre-pass output ([batch][dev]).
template <int KIND, int GROUP, int QUAD, bool XF, bool PAIRS = false>
__device__ __forceinline__ void quad_rows(const CqJob &J, const CqGeom &geom, float (*T)[QuadShape<KIND, GROUP>::kFloats],
                                          float (*P)[(kQuads - 1) * QuadShape<KIND, GROUP>::kGroups * kRowsPerBlock],
                                          int blk) {
    const int r = threadIdx.x % kRowsPerBlock;
    const int rows = J.rows, batch = J.batch;
    const int tile = blk - J.block_begin;
    const int row = tile * kRowsPerBlock + r;
    const __amdgpu_buffer_rsrc_t codes =
        buffer_rsrc(J.codes + static_cast<size_t>(tile) * geom.chunks * kRowsPerBlock,
                    static_cast<uint32_t>(geom.chunks) * kRowsPerBlock * 16u);
    const __amdgpu_buffer_rsrc_t norms =
        buffer_rsrc(J.norms + static_cast<size_t>(tile) * geom.groups * kRowsPerBlock,
                    static_cast<uint32_t>(geom.groups) * kRowsPerBlock * 2u);
    const int windows = geom.windows, groups = geom.groups;
    const int dev = windows * kWindow;
    const uint32_t mask = KIND == kNib ? 0x3Cu : 0x78u;
    float lut[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) lut[i] = geom.lut[i];

    const int stride = XF ? geom.in : dev;
    // Two activation rows per pass over the codes (the reference pairs tokens,
    // cq.cpp:110-152): each window's chunks are loaded once and feed both rows'
    // tables, row b0 then row b0 + 1 (passes alternate the table and park
    // buffers; quarter 0 adds a pass's parked groups at the next pass, before
    // that row's next window). Per row the order of every operation is that of
    // the one-row loop below, so the outputs are the same bits.
    int b0 = 0;
    for (; PAIRS && b0 + 1 < batch; b0 += 2) {
        const __amdgpu_buffer_rsrc_t rot0 =
            buffer_rsrc(J.act + static_cast<size_t>(b0) * stride, static_cast<uint32_t>(stride) * 4u);
        const __amdgpu_buffer_rsrc_t rot1 =
            buffer_rsrc(J.act + static_cast<size_t>(b0 + 1) * stride, static_cast<uint32_t>(stride) * 4u);
        // activations of pass q = 2 w + row (past the last window: zeros)
        auto act = [&](int q) {
            const __amdgpu_buffer_rsrc_t &rt = (q & 1) ? rot1 : rot0;
            if constexpr (XF) return quad_act_x<KIND, GROUP>(rt, q >> 1, r, geom.scale);
            else return quad_act<KIND>(rt, q >> 1, r);
        };
        QuadState<KIND, GROUP> cur, nxt;
        float2 xr = act(0);
        quad_load<KIND, GROUP>(cur, codes, norms, 0, QUAD, r);
        quad_load<KIND, GROUP>(nxt, codes, norms, 1, QUAD, r);
        __syncthreads();  // the previous rows finished with T[0] and P
        quad_build<KIND, GROUP>(T[0], lut, xr, QUAD, r);
        xr = act(1);
        __syncthreads();
        float sum[2] = {0.0f, 0.0f}, gd = 0.0f;
        // pass (w, row): table T[row], parked P[row]; at its start quarter 0 adds
        // the previous pass's parked groups (the other row's, same or previous
        // window) into that row's sum
        auto pass = [&](auto rowc, QuadState<KIND, GROUP> &st, int w) {
            constexpr int row = decltype(rowc)::value;
            if (QUAD == 0 && (row == 1 || w > 0))
                quad_add_parked<KIND, GROUP>(P[row ^ 1], r, sum[row ^ 1], row == 1 ? w : w - 1, groups);
            quad_compute<KIND, GROUP, QUAD, row == 1>(st, T[row], P[row], r, mask, sum[row], gd, w, groups, codes,
                                                      norms);
            const int q = 2 * w + row;
            quad_build<KIND, GROUP>(T[row ^ 1], lut, xr, QUAD, r);
            xr = act(q + 2);
            __syncthreads();
        };
        const int pairs = windows / 2;
        for (int it = 0; it < pairs; ++it) {
            const int w = 2 * it;
            pass(std::integral_constant<int, 0>{}, cur, w);
            pass(std::integral_constant<int, 1>{}, cur, w);
            pass(std::integral_constant<int, 0>{}, nxt, w + 1);
            pass(std::integral_constant<int, 1>{}, nxt, w + 1);
        }
        if (windows & 1) {
            const int w = windows - 1;
            pass(std::integral_constant<int, 0>{}, cur, w);
            pass(std::integral_constant<int, 1>{}, cur, w);
        }
        if (QUAD == 0) {
            quad_add_parked<KIND, GROUP>(P[1], r, sum[1], windows - 1, groups);
            if (row < rows) {
                ((ND_GLOBAL float *)J.y)[static_cast<size_t>(b0) * rows + row] = sum[0];
                ((ND_GLOBAL float *)J.y)[static_cast<size_t>(b0 + 1) * rows + row] = sum[1];
            }
        }
    }
    for (int b = b0; b < batch; ++b) {
        const __amdgpu_buffer_rsrc_t rot =
            buffer_rsrc(J.act + static_cast<size_t>(b) * stride, static_cast<uint32_t>(stride) * 4u);
        auto act = [&](int w) {
            if constexpr (XF) return quad_act_x<KIND, GROUP>(rot, w, r, geom.scale);
            else return quad_act<KIND>(rot, w, r);
        };
        QuadState<KIND, GROUP> cur, nxt;
        float2 xr = act(0);
        quad_load<KIND, GROUP>(cur, codes, norms, 0, QUAD, r);
        quad_load<KIND, GROUP>(nxt, codes, norms, 1, QUAD, r);
        __syncthreads();  // the previous batch row finished with T[0] and P
        quad_build<KIND, GROUP>(T[0], lut, xr, QUAD, r);
        xr = act(1);
        __syncthreads();
        float sum = 0.0f, gd = 0.0f;
        // Whole window pairs, then the last window if the count is odd; one
        // barrier per window and no condition around any load. Window w is
        // summed from `cur` (even) or `nxt` (odd), whose chunks are refilled
        // with window w + 2 as they are spent; the activations of window
        // w + 1 (loaded one window earlier) then become its table (past the
        // end: zeros, into a buffer nobody reads) and those of window w + 2
        // are requested. Before its own groups of window w quarter 0 adds the
        // other quarters' groups of window w - 1 (P[(w - 1) & 1]).
        const int pairs = windows / 2;
        for (int it = 0; it < pairs; ++it) {
            const int w = 2 * it;
            if (QUAD == 0 && it > 0) quad_add_parked<KIND, GROUP>(P[1], r, sum, w - 1, groups);
            quad_compute<KIND, GROUP, QUAD>(cur, T[0], P[0], r, mask, sum, gd, w, groups, codes, norms);
            quad_build<KIND, GROUP>(T[1], lut, xr, QUAD, r);
            xr = act(w + 2);
            __syncthreads();
            if (QUAD == 0) quad_add_parked<KIND, GROUP>(P[0], r, sum, w, groups);
            quad_compute<KIND, GROUP, QUAD>(nxt, T[1], P[1], r, mask, sum, gd, w + 1, groups, codes, norms);
            quad_build<KIND, GROUP>(T[0], lut, xr, QUAD, r);
            xr = act(w + 3);
            __syncthreads();
        }
        if (windows & 1) {
            const int w = windows - 1;
            if (QUAD == 0 && w > 0) quad_add_parked<KIND, GROUP>(P[1], r, sum, w - 1, groups);
            quad_compute<KIND, GROUP, QUAD>(cur, T[0], P[0], r, mask, sum, gd, w, groups, codes, norms);
            __syncthreads();
        }
        if (QUAD == 0) {
            quad_add_parked<KIND, GROUP>(P[(windows - 1) & 1], r, sum, windows - 1, groups);
            if (row < rows) ((ND_GLOBAL float *)J.y)[static_cast<size_t>(b) * rows + row] = sum;
        }
    }
}

template <int KIND, int GROUP, bool XF>
__global__ __launch_bounds__(kQuadThreads) __attribute__((amdgpu_waves_per_eu(8, 8))) void cq_gemv_quad_kernel(
    CqJob job0, const CqJob *__restrict__ jobs, int njobs, CqGeom geom) {
    using Q = QuadShape<KIND, GROUP>;
    __shared__ __attribute__((aligned(16))) float T[2][Q::kFloats];
    __shared__ float P[2][(kQuads - 1) * Q::kGroups * kRowsPerBlock];
    const int blk = blockIdx.x;
    CqJob J = job0;
    if (njobs > 0) {
        const ND_CONST CqJob *cj = (const ND_CONST CqJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J.codes = cj[j].codes;
        J.norms = cj[j].norms;
        J.act = cj[j].act;
        J.y = cj[j].y;
        J.rows = cj[j].rows;
        J.n_pad = cj[j].n_pad;
        J.block_begin = cj[j].block_begin;
        J.batch = cj[j].batch;
    }
    // one straight-line copy of the window loop per quarter (compile-time
    // table offsets; no mixing of the quarters' load bookkeeping)
    switch (__builtin_amdgcn_readfirstlane(threadIdx.x / kRowsPerBlock)) {
    case 0: quad_rows<KIND, GROUP, 0, XF>(J, geom, T, P, blk); break;
    case 1: quad_rows<KIND, GROUP, 1, XF>(J, geom, T, P, blk); break;
    case 2: quad_rows<KIND, GROUP, 2, XF>(J, geom, T, P, blk); break;
    default: quad_rows<KIND, GROUP, 3, XF>(J, geom, T, P, blk); break;
    }
}

// The quarter GEMV for batches of two or more rows: rows in pairs over one
// pass of the codes (each chunk loaded once for both), an odd last row alone.
// One workgroup per CU (128 VGPRs per lane: the pair loop holds both rows'
// state and the two tables' pipelines). 16 x CQ4 8192^2 g32: batch 2
// 203 -> 181 us, batch 4 403 -> 356 us against one row per pass.
template <int KIND, int GROUP, bool XF>
__global__ __launch_bounds__(kQuadThreads) __attribute__((amdgpu_waves_per_eu(4, 4))) void cq_gemv_quad_pair_kernel(
    CqJob job0, const CqJob *__restrict__ jobs, int njobs, CqGeom geom) {
    using Q = QuadShape<KIND, GROUP>;
    __shared__ __attribute__((aligned(16))) float T[2][Q::kFloats];
    __shared__ float P[2][(kQuads - 1) * Q::kGroups * kRowsPerBlock];
    const int blk = blockIdx.x;
    CqJob J = job0;
    if (njobs > 0) {
        const ND_CONST CqJob *cj = (const ND_CONST CqJob *)(jobs);
        const int j = find_job(cj, njobs, blk);
        J.codes = cj[j].codes;
        J.norms = cj[j].norms;
        J.act = cj[j].act;
        J.y = cj[j].y;
        J.rows = cj[j].rows;
        J.n_pad = cj[j].n_pad;
        J.block_begin = cj[j].block_begin;
        J.batch = cj[j].batch;
    }
    switch (__builtin_amdgcn_readfirstlane(threadIdx.x / kRowsPerBlock)) {
    case 0: quad_rows<KIND, GROUP, 0, XF, true>(J, geom, T, P, blk); break;
    case 1: quad_rows<KIND, GROUP, 1, XF, true>(J, geom, T, P, blk); break;
    case 2: quad_rows<KIND, GROUP, 2, XF, true>(J, geom, T, P, blk); break;
    default: quad_rows<KIND, GROUP, 3, XF, true>(J, geom, T, P, blk); break;
    }
}

// Activation pre-pass of the quarter GEMV: rot[v][0..dev) = per-group FWHT
// of zero-padded x (the reference's transform, cq.cpp:153-156, identical
// butterflies), for nvec = count * batch vectors at once: vector v is row
// v % batch of x0 (xptr null) or of xptr[v / batch] (a device table).
template <int GROUP>
__global__ __launch_bounds__(kRowsPerBlock) void rot_many_kernel(const float *__restrict__ x0,
                                                                 const float *const *__restrict__ xptr, int batch,
                                                                 int in, int dev, float scale, float *__restrict__ rot) {
    static_assert(GROUP <= 64, "in-wave FWHT");
    const int v = blockIdx.y;
    const int p = blockIdx.x * kRowsPerBlock + threadIdx.x;
    const float *xv = (xptr ? xptr[v / batch] : x0) + static_cast<size_t>(v % batch) * in;
    float x[1] = {p < in ? xv[p] : 0.0f};
    window_fwht<GROUP>(x, scale, nullptr);
    if (p < dev) rot[static_cast<size_t>(v) * dev + p] = x[0];
}

// Batches of two or more rows on the 4-bit quarter GEMV take the pair kernel
// (NEEDLE2_GPU_FP32_PAIRS=never: one row per pass). 2-bit matrices keep one
// row per pass: their GEMV is bound by the table lookups, which pairs do not
// reduce, and the pair kernel's one workgroup per CU runs them slower
// (16 x 8192^2 at batch 2: 132 -> 183 us).
static bool pairs_wanted(int max_batch) {
    const char *mode = std::getenv("NEEDLE2_GPU_FP32_PAIRS");
    return max_batch >= 2 && !(mode && std::strcmp(mode, "never") == 0);
}

template <int KIND, bool XF>
void launch_gemv_kind(const CqGeom &g, const CqJob &job0, const CqJob *jobs, int njobs, int blocks, hipStream_t s,
                      int max_batch) {
    dim3 grid(blocks), block(kRowsPerBlock), split(kSplitThreads), quad(kQuadThreads);
    if constexpr (KIND == kNib) {  // (2-bit: LDS-bound, one row per pass)
        if (g.group <= 64 && pairs_wanted(max_batch)) {
            switch (g.group) {
            case 8: hipLaunchKernelGGL((cq_gemv_quad_pair_kernel<KIND, 8, XF>), grid, quad, 0, s, job0, jobs, njobs, g); break;
            case 16: hipLaunchKernelGGL((cq_gemv_quad_pair_kernel<KIND, 16, XF>), grid, quad, 0, s, job0, jobs, njobs, g); break;
            case 32: hipLaunchKernelGGL((cq_gemv_quad_pair_kernel<KIND, 32, XF>), grid, quad, 0, s, job0, jobs, njobs, g); break;
            default: hipLaunchKernelGGL((cq_gemv_quad_pair_kernel<KIND, 64, XF>), grid, quad, 0, s, job0, jobs, njobs, g); break;
            }
            ND_HIP(hipGetLastError());
            return;
        }
    }
    switch (g.group > kWindow ? 0 : g.group) {
    case 8: hipLaunchKernelGGL((cq_gemv_quad_kernel<KIND, 8, XF>), grid, quad, 0, s, job0, jobs, njobs, g); break;
    case 16: hipLaunchKernelGGL((cq_gemv_quad_kernel<KIND, 16, XF>), grid, quad, 0, s, job0, jobs, njobs, g); break;
    case 32: hipLaunchKernelGGL((cq_gemv_quad_kernel<KIND, 32, XF>), grid, quad, 0, s, job0, jobs, njobs, g); break;
    case 64: hipLaunchKernelGGL((cq_gemv_quad_kernel<KIND, 64, XF>), grid, quad, 0, s, job0, jobs, njobs, g); break;
    case 128:
        if (wsplit_wanted(g))
            hipLaunchKernelGGL((cq_gemv_wsplit_kernel<KIND, 128>), grid, dim3(kWsplitThreads), 0, s, job0, jobs, njobs, g);
        else
            hipLaunchKernelGGL((cq_gemv_split_kernel<KIND, 128>), grid, split, 0, s, job0, jobs, njobs, g);
        break;
    case 256: hipLaunchKernelGGL((cq_gemv_kernel<KIND, 256>), grid, block, 0, s, job0, jobs, njobs, g); break;
    default: hipLaunchKernelGGL((cq_gemv_kernel<KIND, 0>), grid, block, 0, s, job0, jobs, njobs, g); break;
    }
    ND_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Row dequantization (cq.cpp:276-284): tmp = cb[code]*half(norm), then FWHT.
// ---------------------------------------------------------------------------
__global__ void dequant_rows_kernel(CqGeom geom, const uint4 *__restrict__ codes, const uint16_t *__restrict__ norms,
                                    const int64_t *__restrict__ ids, int padded, float *__restrict__ tmp,
                                    int tmp_stride) {
    int p = blockIdx.x * blockDim.x + threadIdx.x;
    int i = blockIdx.y;
    if (p >= padded) return;
    const int row = static_cast<int>(ids[i]);
    const int cpc = geom.kind == kNib ? 32 : 64;
    const int c = p / cpc, within = p % cpc;
    const uint4 v = codes[code_index(row, c, geom.chunks)];
    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
    unsigned code;
    if (geom.kind == kNib) code = (words[within >> 3] >> ((within & 7) * 4)) & 15u;
    else code = (words[within >> 4] >> ((within & 15) * 2)) & 3u;
    const float norm = h2f(norms[norm_index(row, p / geom.group, geom.groups)]);
    tmp[static_cast<size_t>(i) * tmp_stride + p] = geom.lut[code] * norm;
}

// Plain streaming copy (16 B per lane per step): the reference point for
// scaling hardware byte counters to HBM bytes.
__global__ __launch_bounds__(256) void copy_kernel(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst, size_t n) {
    size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (; i < n; i += stride) dst[i] = src[i];
}

// Candidate rows (engine.cpp:1307-1349 projects only the candidate rows of
// the LM head): output row i of a compact device-layout matrix of n_pad rows
// takes the codes and norms of row ids[i]. Rows past `count` are zero; an id
// outside [0, rows) gets zero codes and NaN norms, so its output is NaN.
// Grid: x over output rows (one per lane), y strides over chunks and groups.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint4 *__restrict__ codes,
                                                          const uint16_t *__restrict__ norms, int rows, int chunks,
                                                          int groups, const int32_t *__restrict__ ids, int count,
                                                          uint4 *__restrict__ out_codes, uint16_t *__restrict__ out_norms) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int id = i < count ? ids[i] : 0;
    const bool real = i < count && id >= 0 && id < rows;
    const uint16_t fill = i < count ? 0x7E00 : 0;  // fp16 NaN for an invalid id
    for (int c = blockIdx.y; c < chunks; c += gridDim.y)
        out_codes[code_index(i, c, chunks)] = real ? codes[code_index(id, c, chunks)] : make_uint4(0, 0, 0, 0);
    for (int g = blockIdx.y; g < groups; g += gridDim.y)
        out_norms[norm_index(i, g, groups)] = real ? norms[norm_index(id, g, groups)] : fill;
}

// y[b][i] = full[b][ids[i]] for b < batch (NaN for an id outside [0, rows)).
__global__ __launch_bounds__(256) void gather_outputs_kernel(const float *__restrict__ full, int rows,
                                                             const int32_t *__restrict__ ids, int count,
                                                             float *__restrict__ y) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int b = blockIdx.y;
    if (i >= count) return;
    const int id = ids[i];
    y[static_cast<size_t>(b) * count + i] =
        id >= 0 && id < rows ? full[static_cast<size_t>(b) * rows + id] : __builtin_nanf("");
}

}  // namespace

void launch_copy(const void *src, void *dst, size_t bytes, hipStream_t s) {
    const size_t n = bytes / 16;
    if (!n) return;
    hipLaunchKernelGGL(copy_kernel, dim3(4096), dim3(256), 0, s, static_cast<const u32x4 *>(src),
                       static_cast<u32x4 *>(dst), n);
    ND_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
void launch_relayout(const uint8_t *packed, int rows, int rowbytes, int bits, int padded, uint4 *codes, int n_pad,
                     int chunks, hipStream_t s) {
    dim3 grid((n_pad + 255) / 256, chunks), block(256);
    hipLaunchKernelGGL(relayout_kernel, grid, block, 0, s, packed, rows, rowbytes, bits, padded, codes, n_pad, chunks);
    ND_HIP(hipGetLastError());
}

void launch_norms_transpose(const uint16_t *norms, int rows, int groups, uint16_t *out, int n_pad, hipStream_t s) {
    dim3 grid((n_pad + 255) / 256, groups), block(256);
    hipLaunchKernelGGL(norms_transpose_kernel, grid, block, 0, s, norms, rows, groups, out, n_pad);
    ND_HIP(hipGetLastError());
}

static constexpr int kMaxLdsGroup = 16384;

static void transform_impl(const float *x, int x_stride, float *rot, int rot_stride, int nvec, int in, int padded,
                           int out_limit, int group, float scale, hipStream_t s, float *scratch) {
    if (nvec <= 0) return;
    if (group <= kMaxLdsGroup) {
        int seg = group > 1024 ? group : 1024;
        dim3 grid((out_limit + seg - 1) / seg, nvec), block(256);
        hipLaunchKernelGGL(transform_kernel, grid, block, seg * sizeof(float), s, x, x_stride, rot, rot_stride, in,
                           padded, out_limit, group, scale, seg);
        ND_HIP(hipGetLastError());
        return;
    }
    // large groups: stage through a padded scratch copy in global memory
    ND_CHECK(scratch != nullptr, "internal: FWHT scratch missing for large group");
    dim3 block(256);
    dim3 gcopy((padded + 255) / 256, nvec);
    hipLaunchKernelGGL(pad_copy_kernel, gcopy, block, 0, s, x, x_stride, scratch, padded, in, padded);
    dim3 gst((padded / 2 + 255) / 256, nvec);
    for (int h = 1; h < group; h <<= 1)
        hipLaunchKernelGGL(butterfly_stage_kernel, gst, block, 0, s, scratch, padded, padded, h);
    dim3 gout((out_limit + 255) / 256, nvec);
    hipLaunchKernelGGL(scale_crop_kernel, gout, block, 0, s, scratch, padded, rot, rot_stride, padded, out_limit,
                       scale);
    ND_HIP(hipGetLastError());
}

void launch_transform(const float *x, int x_stride, float *rot, int rot_stride, int nvec, int in, int padded,
                      int dev_positions, int group, float scale, hipStream_t s) {
    // Large groups need scratch; callers of this entry point guarantee
    // group <= kMaxLdsGroup (larger groups go through launch_transform_big).
    transform_impl(x, x_stride, rot, rot_stride, nvec, in, padded, dev_positions, group, scale, s, nullptr);
}

void launch_transform_big(const float *x, int x_stride, float *rot, int rot_stride, int nvec, int in, int padded,
                          int out_limit, int group, float scale, float *scratch, hipStream_t s) {
    transform_impl(x, x_stride, rot, rot_stride, nvec, in, padded, out_limit, group, scale, s, scratch);
}

void launch_rot_many(const float *x0, const float *const *xptr, int batch, int nvec, int in, int dev, int group,
                     float scale, float *rot, hipStream_t s) {
    if (nvec <= 0) return;
    dim3 grid(dev / kRowsPerBlock, nvec), block(kRowsPerBlock);
    switch (group) {
    case 8: hipLaunchKernelGGL(rot_many_kernel<8>, grid, block, 0, s, x0, xptr, batch, in, dev, scale, rot); break;
    case 16: hipLaunchKernelGGL(rot_many_kernel<16>, grid, block, 0, s, x0, xptr, batch, in, dev, scale, rot); break;
    case 32: hipLaunchKernelGGL(rot_many_kernel<32>, grid, block, 0, s, x0, xptr, batch, in, dev, scale, rot); break;
    case 64: hipLaunchKernelGGL(rot_many_kernel<64>, grid, block, 0, s, x0, xptr, batch, in, dev, scale, rot); break;
    default: throw Error("internal: activation pre-pass takes groups of 8 .. 64");
    }
    ND_HIP(hipGetLastError());
}

// The in-kernel transform repeats the group FWHT in every workgroup and quarter
// (about +18% GEMV time on 8192-wide inputs, +7% on 512-wide ones), so it only
// pays where saving the pre-pass launch outweighs that: inputs of at most two
// windows (the 8192 x 512 device call: 10.2 -> 6.7 us). NEEDLE2_GPU_FP32_XF =
// always / never overrides.
bool gemv_quad_takes_x(int group, int in) {
    if (group > 64) return false;
    const char *mode = std::getenv("NEEDLE2_GPU_FP32_XF");
    if (mode && std::strcmp(mode, "never") == 0) return false;
    if (mode && std::strcmp(mode, "always") == 0) return true;
    return in <= 2 * kWindow;
}

void launch_cq_gemv(const CqGeom &g, const CqJob &job0, const CqJob *jobs, int njobs, int blocks, hipStream_t s,
                    bool x_raw, int max_batch) {
    if (blocks <= 0) return;
    ND_CHECK(!x_raw || g.group <= 64, "internal: raw GEMV input for a group the pre-pass does not serve");
    if (x_raw) {
        if (g.kind == kNib) launch_gemv_kind<kNib, true>(g, job0, jobs, njobs, blocks, s, max_batch);
        else launch_gemv_kind<kCrumb, true>(g, job0, jobs, njobs, blocks, s, max_batch);
        return;
    }
    if (g.kind == kNib) launch_gemv_kind<kNib, false>(g, job0, jobs, njobs, blocks, s, max_batch);
    else launch_gemv_kind<kCrumb, false>(g, job0, jobs, njobs, blocks, s, max_batch);
}

void launch_gather_rows(const uint4 *codes, const uint16_t *norms, int rows, int chunks, int groups,
                        const int32_t *ids, int count, int n_pad, uint4 *out_codes, uint16_t *out_norms, hipStream_t s) {
    if (count <= 0) return;
    dim3 grid(n_pad / 256, std::min(std::max(chunks, groups), 64)), block(256);
    hipLaunchKernelGGL(gather_rows_kernel, grid, block, 0, s, codes, norms, rows, chunks, groups, ids, count,
                       out_codes, out_norms);
    ND_HIP(hipGetLastError());
}

void launch_gather_outputs(const float *full, int rows, const int32_t *ids, int count, int batch, float *y,
                           hipStream_t s) {
    if (count <= 0 || batch <= 0) return;
    dim3 grid((count + 255) / 256, batch), block(256);
    hipLaunchKernelGGL(gather_outputs_kernel, grid, block, 0, s, full, rows, ids, count, y);
    ND_HIP(hipGetLastError());
}

void launch_cq_rows(const CqGeom &g, const uint4 *codes, const uint16_t *norms, const int64_t *ids,
                    int count, int in, int padded, float *scratch, float *y, hipStream_t s) {
    if (count <= 0) return;
    dim3 grid((padded + 255) / 256, count), block(256);
    hipLaunchKernelGGL(dequant_rows_kernel, grid, block, 0, s, g, codes, norms, ids, padded, scratch, padded);
    ND_HIP(hipGetLastError());
    // in-place FWHT of scratch rows, cropped to `in` columns into y
    float scale = g.scale;
    if (g.group <= kMaxLdsGroup) {
        transform_impl(scratch, padded, y, in, count, padded, padded, in, g.group, scale, s, nullptr);
    } else {
        dim3 gst((padded / 2 + 255) / 256, count);
        for (int h = 1; h < g.group; h <<= 1)
            hipLaunchKernelGGL(butterfly_stage_kernel, gst, block, 0, s, scratch, padded, padded, h);
        dim3 gout((in + 255) / 256, count);
        hipLaunchKernelGGL(scale_crop_kernel, gout, block, 0, s, scratch, padded, y, in, padded, in, scale);
        ND_HIP(hipGetLastError());
    }
}

}  // namespace nd
