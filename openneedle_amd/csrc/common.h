// Shared host/device definitions for the gfx950 CQ library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace nd {

// ---------------------------------------------------------------------------
// Errors: every entry point converts exceptions into the reference's error
// channels (NULL / -1 / NaN-poisoned outputs) plus a thread-local message.
// ---------------------------------------------------------------------------
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void set_error(const std::string &msg);
const char *get_error();

[[noreturn]] void hip_fail(const char *expr, hipError_t e, const char *file, int line);

#define ND_HIP(expr)                                                   \
    do {                                                               \
        hipError_t nd_e_ = (expr);                                     \
        if (nd_e_ != hipSuccess) nd::hip_fail(#expr, nd_e_, __FILE__, __LINE__); \
    } while (0)

// Waits for the stream by polling it instead of hipStreamSynchronize, whose
// wake-up measured 2-10% of an engine decode step (~650 us of kernels that end
// by writing pinned host memory); the host thread spins while the stream runs.
// Calls that end with an asynchronous device-to-host copy measured slower with
// it (a 2048 x 512 host-pointer GEMV: 23 -> 27-31 us) and keep
// hipStreamSynchronize.
inline void wait_stream(hipStream_t s) {
    for (hipError_t q = hipStreamQuery(s); q != hipSuccess; q = hipStreamQuery(s))
        if (q != hipErrorNotReady) ND_HIP(q);
}

#define ND_CHECK(cond, msg)                        \
    do {                                           \
        if (!(cond)) throw nd::Error(msg);         \
    } while (0)

// ---------------------------------------------------------------------------
// Owning device / pinned-host buffers.
// ---------------------------------------------------------------------------
template <class T>
struct DevBuf {
    T *p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    ~DevBuf() { release(); }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    // Grow-only allocation; contents are not preserved.
    void reserve(size_t count) {
        if (count <= n && p) return;
        release();
        ND_HIP(hipMalloc(reinterpret_cast<void **>(&p), (count ? count : 1) * sizeof(T)));
        n = count;
    }
};

template <class T>
struct HostBuf {
    T *p = nullptr;
    size_t n = 0;
    HostBuf() = default;
    HostBuf(const HostBuf &) = delete;
    HostBuf &operator=(const HostBuf &) = delete;
    ~HostBuf() { release(); }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        n = 0;
    }
    void reserve(size_t count) {
        if (count <= n && p) return;
        release();
        ND_HIP(hipHostMalloc(reinterpret_cast<void **>(&p), (count ? count : 1) * sizeof(T), hipHostMallocDefault));
        n = count;
    }
};

// ---------------------------------------------------------------------------
// Device layout of a CQ matrix.
//
// Codes are re-laid out at create time into row tiles of kRowsPerBlock rows,
// chunk-major inside a tile: a chunk is 16 bytes of one row (32 four-bit
// codes or 64 two-bit codes), one uint4 per (chunk, row) at code_index(), so
// the 64 lanes of a wavefront, one row each, read 1 KiB contiguous per chunk
// and a workgroup's whole tile is one contiguous run. Norms are fp16 at
// norm_index(). Rows are padded to a multiple of kRowsPerBlock with zero
// codes/norms; each row's codes are padded to a whole number of table
// windows (kWindow positions) with zero codes.
// CQ4 and CQ3 use 4-bit device codes (CQ3 is widened once at create time);
// CQ2 and ternary use 2-bit device codes.
// ---------------------------------------------------------------------------
// Address-space qualifiers for device code: pointers read out of job
// descriptors are cast so loads compile to global_* (not flat_*) and
// wave-uniform activations to scalar s_load_*.
#define ND_GLOBAL __attribute__((address_space(1)))
#define ND_CONST __attribute__((address_space(4)))

// 16-byte code chunk as a clang vector (trivially copyable from any address space)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Raw buffer resource over [base, base + bytes): loads take a wave-uniform
// soffset plus one per-lane voffset, and offsets >= bytes read as zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// Cache policy of the GEMV kernels' weight-code loads: non-temporal ("nt",
// the buffer load's cache-policy bit 1). Each code chunk is read once per
// call, and every load instruction reads whole lines (a wave's lanes cover
// contiguous 16-byte pieces). On MI355X a streaming probe of the GEMVs'
// pattern (512 workgroups, each walking its own 1.18 MB row tile) read
// 604 MB in 101 us with plain loads and in 88.6 us with nt ones (plain
// grid-stride streaming: 86 us); the 16 x CQ4 8192 x 8192 GEMV went from
// 111-112 to 104-106 us, the int8 batch-1 stack from 108 to 95 us. Norm
// loads (2 bytes per lane) keep the default policy (measured slightly
// slower with nt), and so do the attention's K / V rows, whose lanes read
// each 64-byte row in four 16-byte pieces (24.7 -> 30.4 us with nt).
constexpr int kStreamLoad = 2;

#ifndef ND_ROWS
#define ND_ROWS 256
#endif
#ifndef ND_WINDOW
#define ND_WINDOW 256
#endif
constexpr int kRowsPerBlock = ND_ROWS;  // rows per workgroup (one per lane)
constexpr int kWindow = ND_WINDOW;      // code positions per LDS table window
static_assert(kRowsPerBlock >= 64 && kWindow % kRowsPerBlock == 0 && kWindow % 64 == 0, "window/block geometry");

enum CodeKind : int { kNib = 0, kCrumb = 1 };

struct CqGeom {
    int kind;        // kNib or kCrumb
    int group;       // group size (power of two >= 8)
    int groups;      // real groups per row (padded / group)
    int windows;     // table windows per row (device positions / kWindow)
    int chunks;      // 16-byte chunks per row in the device layout
    int in;          // input length (x row stride when the FWHT is fused)
    float scale;     // 1/sqrt(group), computed on the host as the reference does
    float lut[16];   // fp32 codebook indexed by device code
};

// Device layout of one matrix: rows in tiles of kRowsPerBlock (one GEMV
// workgroup each); inside a tile, chunk-major with one 16-byte chunk per row:
//   codes[tile][chunk][kRowsPerBlock]   norms[tile][group][kRowsPerBlock]
// A workgroup therefore streams one contiguous run of chunks * 4 KiB of codes
// (and groups * 512 B of norms), which HBM serves faster than the same bytes
// strided across the whole matrix.
__host__ __device__ inline size_t code_index(int r, int c, int chunks) {
    return (static_cast<size_t>(r / kRowsPerBlock) * chunks + c) * kRowsPerBlock + r % kRowsPerBlock;
}
__host__ __device__ inline size_t norm_index(int r, int g, int groups) {
    return (static_cast<size_t>(r / kRowsPerBlock) * groups + g) * kRowsPerBlock + r % kRowsPerBlock;
}

// Groups of 128 and 256 run the activation FWHT inside the FP32 GEMV kernel.
// Groups up to 64 take a batched pre-pass (launch_rot_many) ahead of the
// quarter-split GEMV; groups above one window use the generic transform pass.
inline bool gemv_fuses_fwht(int group) { return group > 64 && group <= kWindow; }

// Largest group the int8 path's one-launch prepare (FWHT + quantize in LDS) takes.
constexpr int kSdotFusedPrepareMaxGroup = 16384;
inline bool gemv_prepass(int group) { return group <= 64; }

struct CqJob {
    const uint4 *codes;       // [n_pad / kRowsPerBlock][chunks][kRowsPerBlock]
    const uint16_t *norms;    // [n_pad / kRowsPerBlock][groups][kRowsPerBlock]
    const float *act;         // x [batch][in] (fused FWHT) or rot [batch][windows*kWindow]
    float *y;                 // outputs [batch][rows]
    int rows;
    int n_pad;
    int block_begin;          // first workgroup index of this job
    int batch;
};

// int8 ("SDOT") path: same code layout, activations pre-quantized.
struct SdotGeom {
    int kind, group, groups, windows, chunks;
    float centroid_scale;     // cs = max|cb|/127
    uint32_t cent[4];         // int8 centroids packed little-endian (16 entries)
    int in, padded;           // input length, padded to whole groups
    float scale;              // 1/sqrt(group), as the prepare uses it
};

struct SdotJob {
    const uint4 *codes;
    const uint16_t *norms;
    const int32_t *q;         // permuted int8 activations [batch][windows*kWindow/4]
    const float *xs;          // per-group activation scales [batch][groups]
    float *y;
    int rows, n_pad, block_begin, batch;
    const float *xst;         // the same scales transposed, [groups][batch] (MFMA path; null: dot4 path only)
    int ystride;              // floats between batch rows of y (0: rows)
    const float *x;           // the fp32 input row (batch 1), for launch_sdot_gemv_x
};

// Where a kernel that produces the next int8 projection's input leaves it
// prepared (the prepare kernel's outputs): q [batch][dev] permuted codes, xs
// [batch][groups] and xst [groups][batch] scales, for groups of 32 positions.
// q null: nothing to prepare.
struct PrepOut {
    int8_t *q;
    float *xs, *xst;
    int dev, padded, groups, kind, batch;
    float scale;
};

// Chained int8 plans (abi.cpp): where a producer of `x` ([batch][n] on the
// device) may leave next_plan's input prepared (q null: next_plan's group is
// not 32; a plan that does not read exactly x is an error); whether
// next_plan wants it prepared at all (false: its GEMV prepares its own
// input); next_plan's own prepare launch, marking the input as left; and the
// mark alone, after a producer kernel filled `plan_prep_target`.
PrepOut plan_prep_target(const void *next_plan, const float *x, int n, int batch);
bool plan_wants_input(const void *next_plan);
void plan_prepare_input(void *next_plan, hipStream_t s);
void plan_mark_staged(void *next_plan);

// ---------------------------------------------------------------------------
// Kernel launchers (implemented in the .hip files).
// ---------------------------------------------------------------------------

// Re-lay out row-major packed codes (rowbytes per row) into the device layout.
// bits: 2, 3, 4 or 5 (ternary); CQ3 is widened to 4-bit codes.
void launch_relayout(const uint8_t *packed, int rows, int rowbytes, int bits, int padded,
                     uint4 *codes, int n_pad, int chunks, hipStream_t s);
void launch_norms_transpose(const uint16_t *norms, int rows, int groups, uint16_t *out, int n_pad, hipStream_t s);

// rot[v][0..dev) = FWHT per group of zero-padded x[v][0..in), for nvec vectors.
void launch_transform(const float *x, int x_stride, float *rot, int rot_stride, int nvec, int in,
                      int padded, int dev_positions, int group, float scale, hipStream_t s);

// rot[v][0..dev) = per-group FWHT of zero-padded x for nvec vectors (groups
// of 8 .. 64): vector v is row v % batch of x0 (xptr null) or of xptr[v / batch].
void launch_rot_many(const float *x0, const float *const *xptr, int batch, int nvec, int in, int dev, int group,
                     float scale, float *rot, hipStream_t s);

// njobs == 0: one job passed by value (job0); otherwise jobs_dev[0..njobs). x_raw (groups <= 64): the jobs'
// act is the raw input [batch][in], which the GEMV transforms itself (no launch_rot_many). max_batch: the
// largest job batch (groups <= 64 take two activation rows per pass over the codes from 2 on).
void launch_cq_gemv(const CqGeom &g, const CqJob &job0, const CqJob *jobs_dev, int njobs, int total_blocks,
                    hipStream_t s, bool x_raw = false, int max_batch = 1);
// Whether callers give a group <= 64 GEMV of input width `in` the raw input instead of the pre-pass output.
bool gemv_quad_takes_x(int group, int in);

// Dequantize rows: y[i][0..in) = FWHT(cb[code]*norm) cropped; uses rot-sized scratch.
// Candidate rows: output row i (< count) of a compact device-layout matrix of
// n_pad rows (a multiple of kRowsPerBlock) holds row ids[i] of the source;
// rows past count are zero, an id outside [0, rows) gets NaN norms.
void launch_gather_rows(const uint4 *codes, const uint16_t *norms, int rows, int chunks, int groups,
                        const int32_t *ids, int count, int n_pad, uint4 *out_codes, uint16_t *out_norms, hipStream_t s);
// y[b][i] = full[b][ids[i]] over batch rows (NaN for an id outside [0, rows)).
void launch_gather_outputs(const float *full, int rows, const int32_t *ids, int count, int batch, float *y,
                           hipStream_t s);
void launch_cq_rows(const CqGeom &g, const uint4 *codes, const uint16_t *norms, const int64_t *ids, int count, int in, int padded, float *scratch, float *y,
                    hipStream_t s);

// int8 path, one launch for nvec = count * batch vectors: vector v is row
// v % batch of matrix input v / batch, read from x0 (count == 1, xptr null) or
// xptr[v / batch] (a device table); each row has `in` floats. FWHT per group,
// quantize, permute. Returns false (nothing launched) when the group is too
// large for one block's LDS; callers then transform and quantize separately.
// xst (nullable) also receives the scales transposed per matrix input: [v / batch][groups][v % batch].
bool launch_sdot_prepare(const float *x0, const float *const *xptr, int batch, int nvec, int in, int padded,
                         int dev_positions, int group, float scale, int kind, int32_t *q, float *xs, float *xst,
                         hipStream_t s);
// int8 path: quantize rot (already transformed) into permuted int8 + scales.
void launch_sdot_quantize(const float *rot, int rot_stride, int nvec, int padded, int dev_positions,
                          int group, int kind, int32_t *q, float *xs, hipStream_t s);
// The batch (uniform across jobs) is processed in tiles that decode each code once.
void launch_sdot_gemv(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs_dev, int njobs, int total_blocks,
                      int batch, hipStream_t s);
// As launch_sdot_gemv for the K-split kernel's shapes (small matrices, batch
// 2 and more, groups 32 .. 256), with 32-row workgroups whose outputs of each
// batch row, one group of 32 positions of the next projection's input, are
// also left prepared in `po` (a single job whose rows are that input's
// positions). False, with nothing launched, for other shapes.
bool launch_sdot_gemv_prep(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs_dev, int njobs,
                           int total_blocks, int batch, const PrepOut &po, hipStream_t s);
// Batch 1 on the small-matrix K-split kernel, which then prepares each job's input row (job.x) itself
// (the prepare kernels' arithmetic) instead of reading q / xs: true when launch_sdot_gemv would run that
// kernel for this shape and the prepared row fits its LDS (NEEDLE2_GPU_INT8_XIN=never: always false).
bool sdot_gemv_takes_x(const SdotGeom &g, int blocks, int batch);
void launch_sdot_gemv_x(const SdotGeom &g, const SdotJob &job0, const SdotJob *jobs_dev, int njobs, int total_blocks,
                        hipStream_t s);
// The same products' int32 group dots, dots[b][row][g], from the kernels the GEMV runs for this batch on a
// large matrix (batch 1: the row kernel; 2 or more: the 4 x 4 x 4 batch-tile kernel); one job only.
void launch_sdot_dots(const SdotGeom &g, const SdotJob &job0, int total_blocks, int batch, int32_t *dots,
                      hipStream_t s);

}  // namespace nd
