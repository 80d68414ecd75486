// Host-side objects behind the C ABI.
#pragma once

#include "common.h"

namespace nd {

void launch_transform_big(const float *x, int x_stride, float *rot, int rot_stride, int nvec, int in, int padded,
                          int out_limit, int group, float scale, float *scratch, hipStream_t s);

void launch_copy(const void *src, void *dst, size_t bytes, hipStream_t s);
// calibration (calib_kernels.hip)
float calib_launch_us(int launches, hipStream_t s);
void calib_lds(int width, float *bytes_per_clk_per_cu, float *ghz, hipStream_t s);
float calib_stream_us(const void *src, size_t bytes, int pattern, hipStream_t s);

// fp16 activations of the prefill GEMM in MFMA fragment order: m rounded up to 32 rows
size_t prefill_xf_halves(int m, int dev);
void launch_prefill_transform(const float *x, int m, int in, int padded, int dev, int group, float scale,
                              _Float16 *xf, hipStream_t s);
// codes4: the matrix's codes as 4-bit device codes (chunks4 = dev / 32 chunks per row tile row)
void launch_prefill_gemm(const CqGeom &geom, const uint4 *codes4, int chunks4, const uint16_t *norms, int rows,
                         const _Float16 *xf, int m, int dev, int padded, const uint16_t *cb_half, float *y,
                         hipStream_t s);
// 2-bit device codes of n_pad rows -> the same positions as 4-bit device codes (for the prefill GEMM)
void launch_widen_crumbs(const uint4 *codes2, int chunks2, int n_pad, uint4 *codes4, hipStream_t s);

// Runs f, converting exceptions into -1 plus the thread-local message. The
// message is cleared first so a non-empty needle2_gpu_error() after a call
// always belongs to that call.
template <class F>
int guarded(F &&f) {
    set_error("");
    try {
        f();
        return 0;
    } catch (const std::exception &e) {
        set_error(e.what());
    } catch (...) {
        set_error("unknown error");
    }
    return -1;
}

// A CQ matrix resident in device memory (layout described in common.h).
struct Matrix {
    int out = 0, in = 0, bits = 0, group = 0, padded = 0, groups = 0, rowbytes = 0;
    int kind = kNib, windows = 0, dev = 0, chunks = 0, n_pad = 0;
    float scale = 1.0f;
    float lut[16] = {};
    float cb_raw[16] = {};
    DevBuf<uint4> codes;
    DevBuf<uint16_t> norms;

    // packed [out][rowbytes] and norms [out][groups] in host memory (copied, then waited for), or with
    // `device_inputs` in device memory (read by the relayout kernels on `s`; nothing waited for).
    void upload(const uint8_t *packed, const uint16_t *norms, int out, int in, int bits, int group, const float *cb,
                hipStream_t s, bool device_inputs = false);
    CqGeom geom() const;
    // rot[v] = FWHT(x[v]) over dev positions for nvec vectors.
    void transform(const float *x, int x_stride, float *rot, int nvec, DevBuf<float> &big, hipStream_t s) const;
};

// Per-handle stream (created on first use: creating one costs ~150 us, and
// device-resident callers pass their own) and grow-only staging buffers.
struct Staging {
    hipStream_t stream();
    DevBuf<float> x, rot, y, big, xs, xst;
    DevBuf<int32_t> q;
    DevBuf<_Float16> xh;  // fp16 transformed activations of the prefill GEMM
    DevBuf<uint4> gcodes;   // candidate rows gathered into a compact matrix
    DevBuf<uint16_t> gnorms;
    DevBuf<int32_t> ids;
    DevBuf<float> yfull;    // all outputs, when most rows are candidates
    HostBuf<float> hx, hy;
    HostBuf<int32_t> hids;
    DevBuf<uint8_t> jobs;   // per-call job tables (needle2_cq_linear_many)
    HostBuf<uint8_t> hjobs;
    Staging() = default;
    ~Staging();
    Staging(const Staging &) = delete;
    Staging &operator=(const Staging &) = delete;

  private:
    hipStream_t stream_ = nullptr;
};

// The FP32 GEMV over rows [0, rows) of a device-layout matrix with m's
// geometry (codes / norms: m's own or a compact copy), staging in `st`.
void matrix_gemv(const Matrix &m, Staging &st, const uint4 *codes, const uint16_t *norms, int rows, int n_pad,
                 const float *d_x, float *d_y, int batch, hipStream_t s);

// Rows ids[0..count) of a matrix as a compact matrix of n_pad rows (gathered
// into st.gcodes / st.gnorms), or none when most rows are asked for.
struct Candidates {
    const uint4 *codes = nullptr;
    const uint16_t *norms = nullptr;
    int n_pad = 0;
    bool full = false;  // run the whole matrix, then pick the outputs
};
Candidates gather_candidates(const Matrix &m, Staging &st, const int32_t *d_ids, int count, hipStream_t s);
// Host side of needle2_gpu_*_candidates: checks the ids as the reference does
// (engine.cpp:1302-1306), then copies them to st.ids.
void upload_candidates(Staging &st, const int32_t *ids, int count, int rows);

struct CqHandle {
    Matrix m;
    Staging st;
    DevBuf<uint4> codes4;  // 2-bit matrices: the codes widened to 4 bits for the prefill GEMM (built on first use)
    void run_device(const float *d_x, float *d_y, int batch, hipStream_t s);
    // the GEMV over rows [0, rows) of a device-layout matrix with m's geometry
    void gemv(const uint4 *codes, const uint16_t *norms, int rows, int n_pad, const float *d_x, float *d_y, int batch,
              hipStream_t s);
    // d_y[i] = row d_ids[i] of W x for batch-1 x (engine.cpp:1307-1349, the CQ branch)
    void candidates_device(const float *d_x, const int32_t *d_ids, int count, float *d_y, hipStream_t s);
    void candidates_host(const float *x, const int32_t *ids, int count, float *y);
    void linear_host(const float *x, float *y, int batch);
    void rows_host(const int64_t *ids, float *y, int count);
    // prefill GEMM on fp16 MFMA; events (nullable) bracket `repeat` launches of the GEMM kernel
    void gemm_device(const float *d_x, float *d_y, int m, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1,
                     int repeat = 1);
};

// The int8 path's geometry and centroid tables of a CQ matrix (sdot.cpp:35-60).
SdotGeom sdot_geom_of(const Matrix &m);

struct SdotHandle {
    Matrix m;
    Staging st;
    float centroid_scale = 1.0f;
    uint32_t centroids[4] = {};
    void init_tables();
    SdotGeom geom() const;
    void prepare_device(const float *d_x, int batch, int32_t *q, float *xs, float *xst, hipStream_t s);
    void run_device(const float *d_x, float *d_y, int batch, hipStream_t s);
    // d_dots[b][row][g] = the int32 group dots of the int8 product (sdot.cpp:108-137)
    void dots_device(const float *d_x, int32_t *d_dots, int batch, hipStream_t s);
    // d_y[i] = row d_ids[i] of the int8 product for batch-1 x (engine.cpp:1307-1349, the SDOT branch)
    void candidates_device(const float *d_x, const int32_t *d_ids, int count, float *d_y, hipStream_t s);
    void candidates_host(const float *x, const int32_t *ids, int count, float *y);
    void linear_host(const float *x, float *y, int batch);
};

}  // namespace nd
