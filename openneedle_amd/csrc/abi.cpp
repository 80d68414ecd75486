// C ABI of the gfx950 CQ library (libneedle2_native.so).
//
// The first group of exports is the reference's ctypes boundary, with the same
// names, argument meaning, ownership and error behaviour
// (needle2/native.py:124-146; needle2/csrc/cq.cpp:342-371,
// needle2/csrc/sdot.cpp:349-360). The handle uploads the packed codes and
// norms to device memory at create time; linear calls copy x in, run the
// kernels on the handle's stream and copy y out before returning.
// The second group (needle2_gpu_*) is additive: device-resident entry points,
// multi-matrix plans, memory/stream/event helpers and a thread-local error.
#include "abi_internal.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

namespace nd {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string &msg) { g_error = msg; }
const char *get_error() { return g_error.c_str(); }

void hip_fail(const char *expr, hipError_t e, const char *file, int line) {
    throw Error(std::string("HIP error ") + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ") in " + expr +
                " at " + file + ":" + std::to_string(line));
}

static bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// Inputs the kernels cannot run meaningfully are refused at creation (the
// reference's Python loader refuses the same ones before its C call,
// needle2/native.py:190-202): a codebook that is not finite and strictly
// increasing, a norm that is not finite or is below zero (-0 is a zero
// norm), and the reserved ternary crumb 2, which has no centroid.
static void check_codebook(const float *cb, int n) {
    for (int i = 0; i < n; ++i)
        ND_CHECK(std::isfinite(cb[i]) && (i == 0 || cb[i - 1] < cb[i]),
                 "CQ codebook: centroids must be finite and strictly increasing");
}

static void check_norms(const uint16_t *norms, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const uint16_t h = norms[i];
        ND_CHECK((h & 0x7C00u) != 0x7C00u && !((h & 0x8000u) && (h & 0x7FFFu)),
                 "CQ norms: every fp16 group norm must be finite and >= 0");
    }
}

static void check_ternary(const uint8_t *packed, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const uint8_t b = packed[i];
        // crumb value 2 = high bit set, low bit clear
        ND_CHECK(((b >> 1) & ~b & 0x55u) == 0, "CQ ternary codes: crumb value 2 is reserved");
    }
}

// ---------------------------------------------------------------------------
// Matrix upload
// ---------------------------------------------------------------------------
void Matrix::upload(const uint8_t *packed, const uint16_t *host_norms, int out_, int in_, int bits_, int group_,
                    const float *cb, hipStream_t s, bool device_inputs) {
    ND_CHECK(out_ > 0 && in_ > 0, "CQ matrix shape must be positive (rows and columns)");
    ND_CHECK(bits_ == 2 || bits_ == 3 || bits_ == 4 || bits_ == 5, "CQ bits must be 2, 3 or 4 (5: ternary crumbs)");
    ND_CHECK(is_pow2(group_) && group_ >= 8, "CQ group must be a power of two of at least 8");
    ND_CHECK(packed && host_norms && cb, "CQ create: null buffer");
    check_codebook(cb, bits_ == 5 ? 3 : 1 << bits_);
    out = out_;
    in = in_;
    bits = bits_;
    group = group_;
    int64_t padded64 = (int64_t(in) + group - 1) / group * group;
    ND_CHECK(padded64 <= std::numeric_limits<int>::max() / 4, "CQ row too long");
    padded = static_cast<int>(padded64);
    groups = padded / group;
    const int storage_bits = bits == 5 ? 2 : bits;
    rowbytes = padded * storage_bits / 8;
    kind = (bits == 2 || bits == 5) ? kCrumb : kNib;
    windows = (padded + kWindow - 1) / kWindow;
    dev = windows * kWindow;
    chunks = dev / (kind == kNib ? 32 : 64);
    n_pad = (out + kRowsPerBlock - 1) / kRowsPerBlock * kRowsPerBlock;
    scale = 1 / std::sqrt(float(group));  // cq.cpp:44
    std::memset(lut, 0, sizeof lut);
    if (bits == 5) {  // ternary crumbs: 3 -> cb[0], 0 -> cb[1], 1 -> cb[2] (cq.cpp:68, 73); 2 is invalid
        lut[0] = cb[1];
        lut[1] = cb[2];
        lut[2] = 0.0f;
        lut[3] = cb[0];
    } else {
        std::memcpy(lut, cb, sizeof(float) * (1u << bits));
    }
    std::memcpy(cb_raw, cb, sizeof(float) * (bits == 5 ? 3 : 1u << bits));
    // host inputs are checked before anything is allocated (device inputs are the caller's to vouch for)
    if (!device_inputs) {
        check_norms(host_norms, size_t(out) * groups);
        if (bits == 5) check_ternary(packed, size_t(out) * rowbytes);
    }

    codes.reserve(size_t(chunks) * n_pad);
    norms.reserve(size_t(groups) * n_pad);
    if (device_inputs) {
        launch_relayout(packed, out, rowbytes, bits, padded, codes.p, n_pad, chunks, s);
        launch_norms_transpose(host_norms, out, groups, norms.p, n_pad, s);
        return;
    }
    DevBuf<uint8_t> raw;
    const size_t raw_bytes = size_t(out) * rowbytes;
    raw.reserve(raw_bytes);
    ND_HIP(hipMemcpyAsync(raw.p, packed, raw_bytes, hipMemcpyHostToDevice, s));
    launch_relayout(raw.p, out, rowbytes, bits, padded, codes.p, n_pad, chunks, s);
    DevBuf<uint16_t> nraw;
    nraw.reserve(size_t(out) * groups);
    ND_HIP(hipMemcpyAsync(nraw.p, host_norms, size_t(out) * groups * 2, hipMemcpyHostToDevice, s));
    launch_norms_transpose(nraw.p, out, groups, norms.p, n_pad, s);
    ND_HIP(hipStreamSynchronize(s));
}

CqGeom Matrix::geom() const {
    CqGeom g{};
    g.kind = kind;
    g.group = group;
    g.groups = groups;
    g.windows = windows;
    g.chunks = chunks;
    g.in = in;
    g.scale = scale;
    std::memcpy(g.lut, lut, sizeof lut);
    return g;
}

void Matrix::transform(const float *x, int x_stride, float *rot, int nvec, DevBuf<float> &big, hipStream_t s) const {
    if (group <= 16384) {
        launch_transform(x, x_stride, rot, dev, nvec, in, padded, dev, group, scale, s);
    } else {
        big.reserve(size_t(nvec) * padded);
        launch_transform_big(x, x_stride, rot, dev, nvec, in, padded, dev, group, scale, big.p, s);
    }
}

hipStream_t Staging::stream() {
    if (!stream_) ND_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
    return stream_;
}
Staging::~Staging() {
    if (stream_) (void)hipStreamDestroy(stream_);
}

// ---------------------------------------------------------------------------
// FP32 handle
// ---------------------------------------------------------------------------
void CqHandle::gemv(const uint4 *codes, const uint16_t *norms, int rows, int n_pad, const float *d_x, float *d_y,
                    int batch, hipStream_t s) {
    matrix_gemv(m, st, codes, norms, rows, n_pad, d_x, d_y, batch, s);
}

void matrix_gemv(const Matrix &m, Staging &st, const uint4 *codes, const uint16_t *norms, int rows, int n_pad,
                 const float *d_x, float *d_y, int batch, hipStream_t s) {
    const float *act = d_x;
    const bool xraw = gemv_prepass(m.group) && gemv_quad_takes_x(m.group, m.in);  // the GEMV transforms x itself
    if (!gemv_fuses_fwht(m.group) && !xraw) {
        st.rot.reserve(size_t(batch) * m.dev);
        if (gemv_prepass(m.group))
            launch_rot_many(d_x, nullptr, batch, batch, m.in, m.dev, m.group, m.scale, st.rot.p, s);
        else
            m.transform(d_x, m.in, st.rot.p, batch, st.big, s);
        act = st.rot.p;
    }
    const CqJob job{codes, norms, act, d_y, rows, n_pad, 0, batch};
    launch_cq_gemv(m.geom(), job, nullptr, 0, n_pad / kRowsPerBlock, s, xraw, batch);
}

void CqHandle::run_device(const float *d_x, float *d_y, int batch, hipStream_t s) {
    if (batch <= 0) return;
    gemv(m.codes.p, m.norms.p, m.out, m.n_pad, d_x, d_y, batch, s);
}

// ---------------------------------------------------------------------------
// Candidate rows (engine.cpp:1307-1349): the same GEMV kernels over a compact
// matrix of the candidate rows, so every output is bit-identical to that row
// of the full product; when at least half the rows are asked for, the full
// GEMV runs and the outputs are picked.
// ---------------------------------------------------------------------------
Candidates gather_candidates(const Matrix &m, Staging &st, const int32_t *d_ids, int count, hipStream_t s) {
    Candidates c;
    if (2 * size_t(count) >= size_t(m.out)) {
        c.full = true;
        return c;
    }
    c.n_pad = (count + kRowsPerBlock - 1) / kRowsPerBlock * kRowsPerBlock;
    st.gcodes.reserve(size_t(c.n_pad) * m.chunks);
    st.gnorms.reserve(size_t(c.n_pad) * m.groups);
    launch_gather_rows(m.codes.p, m.norms.p, m.out, m.chunks, m.groups, d_ids, count, c.n_pad, st.gcodes.p,
                       st.gnorms.p, s);
    c.codes = st.gcodes.p;
    c.norms = st.gnorms.p;
    return c;
}

void upload_candidates(Staging &st, const int32_t *ids, int count, int rows) {
    ND_CHECK(ids && count > 0, "candidates must be nonempty");
    for (int i = 0; i < count; ++i) ND_CHECK(ids[i] >= 0 && ids[i] < rows, "candidate outside vocabulary");
    st.hids.reserve(count);
    st.ids.reserve(count);
    std::memcpy(st.hids.p, ids, size_t(count) * sizeof(int32_t));
    ND_HIP(hipMemcpyAsync(st.ids.p, st.hids.p, size_t(count) * sizeof(int32_t), hipMemcpyHostToDevice, st.stream()));
}

void CqHandle::candidates_device(const float *d_x, const int32_t *d_ids, int count, float *d_y, hipStream_t s) {
    if (count <= 0) return;
    const Candidates c = gather_candidates(m, st, d_ids, count, s);
    if (c.full) {
        st.yfull.reserve(m.out);
        run_device(d_x, st.yfull.p, 1, s);
        launch_gather_outputs(st.yfull.p, m.out, d_ids, count, 1, d_y, s);
    } else {
        gemv(c.codes, c.norms, count, c.n_pad, d_x, d_y, 1, s);
    }
}

void CqHandle::candidates_host(const float *x, const int32_t *ids, int count, float *y) {
    upload_candidates(st, ids, count, m.out);
    st.hx.reserve(m.in);
    st.x.reserve(m.in);
    st.hy.reserve(count);
    st.y.reserve(count);
    std::memcpy(st.hx.p, x, size_t(m.in) * sizeof(float));
    ND_HIP(hipMemcpyAsync(st.x.p, st.hx.p, size_t(m.in) * sizeof(float), hipMemcpyHostToDevice, st.stream()));
    candidates_device(st.x.p, st.ids.p, count, st.y.p, st.stream());
    ND_HIP(hipMemcpyAsync(st.hy.p, st.y.p, size_t(count) * sizeof(float), hipMemcpyDeviceToHost, st.stream()));
    ND_HIP(hipStreamSynchronize(st.stream()));
    std::memcpy(y, st.hy.p, size_t(count) * sizeof(float));
}

void CqHandle::gemm_device(const float *d_x, float *d_y, int m_rows, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1,
                           int repeat) {
    if (m_rows <= 0) return;
    ND_CHECK(prefill_xf_halves(m_rows, m.dev) * 2 < (size_t(1) << 31), "prefill GEMM: m * padded input must be < 2^30");
    const uint4 *c4 = m.codes.p;
    if (m.kind == kCrumb) {  // CQ2 / ternary: the GEMM reads 4-bit codes, widened once
        if (!codes4.p) {
            DevBuf<uint4> wide;
            wide.reserve(size_t(m.n_pad) * m.chunks * 2);
            launch_widen_crumbs(m.codes.p, m.chunks, m.n_pad, wide.p, s);
            // a later call may run on another stream: the copy is published only once it is complete
            ND_HIP(hipStreamSynchronize(s));
            std::swap(codes4.p, wide.p);
            std::swap(codes4.n, wide.n);
        }
        c4 = codes4.p;
    }
    st.xh.reserve(prefill_xf_halves(m_rows, m.dev));
    launch_prefill_transform(d_x, m_rows, m.in, m.padded, m.dev, m.group, m.scale, st.xh.p, s);
    uint16_t cbh[16];
    for (int i = 0; i < 16; ++i) cbh[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(m.lut[i]));
    if (ev0) ND_HIP(hipEventRecord(ev0, s));
    for (int r = 0; r < repeat; ++r)
        launch_prefill_gemm(m.geom(), c4, m.dev / 32, m.norms.p, m.out, st.xh.p, m_rows, m.dev, m.padded, cbh, d_y, s);
    if (ev1) ND_HIP(hipEventRecord(ev1, s));
}

void CqHandle::linear_host(const float *x, float *y, int batch) {
    if (batch <= 0) return;
    const size_t nx = size_t(batch) * m.in, ny = size_t(batch) * m.out;
    st.hx.reserve(nx);
    st.hy.reserve(ny);
    std::memcpy(st.hx.p, x, nx * sizeof(float));
    // The kernels read x straight from the pinned staging buffer where they
    // read each value once (the pre-pass or transform before the GEMV) or the
    // row is at most two windows; a GEMV that transforms a wide row in every
    // workgroup (groups of 128 / 256) reads a device copy. y is written once
    // per value, straight into the pinned buffer. Each host-device copy saved
    // is ~7 us of a CQ4 8192 x 8192 call (80 -> 66 us).
    const bool x_direct = !gemv_fuses_fwht(m.group) || m.in <= 2 * kWindow;
    const float *dx = st.hx.p;
    if (!x_direct) {
        st.x.reserve(nx);
        ND_HIP(hipMemcpyAsync(st.x.p, st.hx.p, nx * sizeof(float), hipMemcpyHostToDevice, st.stream()));
        dx = st.x.p;
    }
    run_device(dx, st.hy.p, batch, st.stream());
    ND_HIP(hipStreamSynchronize(st.stream()));
    std::memcpy(y, st.hy.p, ny * sizeof(float));
}

void CqHandle::rows_host(const int64_t *ids, float *y, int count) {
    if (count <= 0) return;
    for (int i = 0; i < count; ++i) ND_CHECK(ids[i] >= 0 && ids[i] < m.out, "CQ row index outside matrix");
    DevBuf<int64_t> dids;
    dids.reserve(count);
    st.rot.reserve(size_t(count) * m.padded);
    st.y.reserve(size_t(count) * m.in);
    ND_HIP(hipMemcpyAsync(dids.p, ids, size_t(count) * sizeof(int64_t), hipMemcpyHostToDevice, st.stream()));
    launch_cq_rows(m.geom(), m.codes.p, m.norms.p, dids.p, count, m.in, m.padded, st.rot.p, st.y.p,
                   st.stream());
    ND_HIP(hipMemcpyAsync(y, st.y.p, size_t(count) * m.in * sizeof(float), hipMemcpyDeviceToHost, st.stream()));
    ND_HIP(hipStreamSynchronize(st.stream()));
}

// ---------------------------------------------------------------------------
// int8 handle
// ---------------------------------------------------------------------------
SdotGeom sdot_geom_of(const Matrix &m) {
    // sdot.cpp:38-44: cs = max|cb|/127 (1 if zero), centroids = clamp(nearbyint(cb/cs))
    float maximum = 0;
    const int n = 1 << m.bits;
    for (int i = 0; i < n; ++i) maximum = std::max(maximum, std::abs(m.cb_raw[i]));
    SdotGeom g{};
    g.kind = m.kind;
    g.group = m.group;
    g.groups = m.groups;
    g.windows = m.windows;
    g.chunks = m.chunks;
    g.in = m.in;
    g.padded = m.padded;
    g.scale = m.scale;
    g.centroid_scale = maximum > 0 ? maximum / 127 : 1;
    uint8_t cent[16] = {};
    for (int i = 0; i < n; ++i) {
        float v = std::nearbyint(m.cb_raw[i] / g.centroid_scale);
        v = v < -127.0f ? -127.0f : (127.0f < v ? 127.0f : v);
        cent[i] = static_cast<uint8_t>(static_cast<int8_t>(v));
    }
    std::memcpy(g.cent, cent, sizeof g.cent);
    return g;
}

void SdotHandle::init_tables() {
    const SdotGeom g = sdot_geom_of(m);
    centroid_scale = g.centroid_scale;
    std::memcpy(centroids, g.cent, sizeof centroids);
}

SdotGeom SdotHandle::geom() const {
    SdotGeom g = sdot_geom_of(m);
    g.centroid_scale = centroid_scale;
    std::memcpy(g.cent, centroids, sizeof g.cent);
    return g;
}

void SdotHandle::prepare_device(const float *d_x, int batch, int32_t *q, float *xs, float *xst, hipStream_t s) {
    if (launch_sdot_prepare(d_x, nullptr, batch, batch, m.in, m.padded, m.dev, m.group, m.scale, m.kind, q, xs, xst,
                            s))
        return;
    st.rot.reserve(size_t(batch) * m.dev);
    m.transform(d_x, m.in, st.rot.p, batch, st.big, s);
    launch_sdot_quantize(st.rot.p, m.dev, batch, m.padded, m.dev, m.group, m.kind, q, xs, s);
}

void SdotHandle::run_device(const float *d_x, float *d_y, int batch, hipStream_t s) {
    if (batch <= 0) return;
    const SdotGeom g = geom();
    if (sdot_gemv_takes_x(g, m.n_pad / kRowsPerBlock, batch)) {  // the GEMV prepares its input row itself
        SdotJob job{m.codes.p, m.norms.p, nullptr, nullptr, d_y, m.out, m.n_pad, 0, 1, nullptr};
        job.x = d_x;
        launch_sdot_gemv_x(g, job, nullptr, 0, m.n_pad / kRowsPerBlock, s);
        return;
    }
    st.q.reserve(size_t(batch) * m.dev / 4);
    st.xs.reserve(size_t(batch) * m.groups);
    st.xst.reserve(size_t(batch) * m.groups);
    prepare_device(d_x, batch, st.q.p, st.xs.p, st.xst.p, s);
    const SdotJob job{m.codes.p, m.norms.p, st.q.p, st.xs.p, d_y, m.out, m.n_pad, 0, batch, st.xst.p};
    launch_sdot_gemv(geom(), job, nullptr, 0, m.n_pad / kRowsPerBlock, batch, s);
}

void SdotHandle::dots_device(const float *d_x, int32_t *d_dots, int batch, hipStream_t s) {
    if (batch <= 0) return;
    st.q.reserve(size_t(batch) * m.dev / 4);
    st.xs.reserve(size_t(batch) * m.groups);
    st.xst.reserve(size_t(batch) * m.groups);
    prepare_device(d_x, batch, st.q.p, st.xs.p, st.xst.p, s);
    const SdotJob job{m.codes.p, m.norms.p, st.q.p, st.xs.p, nullptr, m.out, m.n_pad, 0, batch, st.xst.p};
    launch_sdot_dots(geom(), job, m.n_pad / kRowsPerBlock, batch, d_dots, s);
}

void SdotHandle::candidates_device(const float *d_x, const int32_t *d_ids, int count, float *d_y, hipStream_t s) {
    if (count <= 0) return;
    const Candidates c = gather_candidates(m, st, d_ids, count, s);
    if (c.full) {
        st.yfull.reserve(m.out);
        run_device(d_x, st.yfull.p, 1, s);
        launch_gather_outputs(st.yfull.p, m.out, d_ids, count, 1, d_y, s);
        return;
    }
    st.q.reserve(m.dev / 4);
    st.xs.reserve(m.groups);
    st.xst.reserve(m.groups);
    prepare_device(d_x, 1, st.q.p, st.xs.p, st.xst.p, s);
    const SdotJob job{c.codes, c.norms, st.q.p, st.xs.p, d_y, count, c.n_pad, 0, 1, st.xst.p};
    launch_sdot_gemv(geom(), job, nullptr, 0, c.n_pad / kRowsPerBlock, 1, s);
}

void SdotHandle::candidates_host(const float *x, const int32_t *ids, int count, float *y) {
    upload_candidates(st, ids, count, m.out);
    st.hx.reserve(m.in);
    st.x.reserve(m.in);
    st.hy.reserve(count);
    st.y.reserve(count);
    std::memcpy(st.hx.p, x, size_t(m.in) * sizeof(float));
    ND_HIP(hipMemcpyAsync(st.x.p, st.hx.p, size_t(m.in) * sizeof(float), hipMemcpyHostToDevice, st.stream()));
    candidates_device(st.x.p, st.ids.p, count, st.y.p, st.stream());
    ND_HIP(hipMemcpyAsync(st.hy.p, st.y.p, size_t(count) * sizeof(float), hipMemcpyDeviceToHost, st.stream()));
    ND_HIP(hipStreamSynchronize(st.stream()));
    std::memcpy(y, st.hy.p, size_t(count) * sizeof(float));
}

void SdotHandle::linear_host(const float *x, float *y, int batch) {
    if (batch <= 0) return;
    const size_t nx = size_t(batch) * m.in, ny = size_t(batch) * m.out;
    // a non-finite value has no int8 code (the reference's loader refuses it, needle2/native.py:249-250)
    for (size_t i = 0; i < nx; ++i) ND_CHECK(std::isfinite(x[i]), "int8 input values must be finite");
    st.hx.reserve(nx);
    st.hy.reserve(ny);
    std::memcpy(st.hx.p, x, nx * sizeof(float));
    // as CqHandle::linear_host: x read in place unless a GEMV that prepares
    // its input in every workgroup would read a wide row many times over
    const bool x_direct = !sdot_gemv_takes_x(geom(), m.n_pad / kRowsPerBlock, batch) || m.in <= 2 * kWindow;
    const float *dx = st.hx.p;
    if (!x_direct) {
        st.x.reserve(nx);
        ND_HIP(hipMemcpyAsync(st.x.p, st.hx.p, nx * sizeof(float), hipMemcpyHostToDevice, st.stream()));
        dx = st.x.p;
    }
    run_device(dx, st.hy.p, batch, st.stream());
    ND_HIP(hipStreamSynchronize(st.stream()));
    std::memcpy(y, st.hy.p, ny * sizeof(float));
}

// ---------------------------------------------------------------------------
// Plans: many matrices of one geometry, one transform and one GEMV launch.
// ---------------------------------------------------------------------------
struct Plan {
    bool sdot = false;
    bool xraw = false;  // FP32, groups <= 64: the GEMV transforms the raw inputs itself
    int count = 0, batch = 1;
    std::vector<CqHandle *> cq;
    std::vector<SdotHandle *> sd;
    std::vector<const float *> xs_in;
    std::vector<float *> ys;
    DevBuf<float> rot;
    DevBuf<int32_t> q;
    DevBuf<float> xscale, xscale_t;
    DevBuf<const float *> xptr;  // device table of the count input pointers (int8 prepare)
    DevBuf<uint8_t> jobs;
    int blocks = 0;
    const Matrix *first = nullptr;
    Staging st;
    bool staged = false;  // a chained producer left this plan's prepared input since its last run
    int inputs = 0;       // distinct int8 inputs prepared per run: 1 when every matrix reads the same x
};

static void plan_upload(Plan &p) {
    const Matrix &m = *p.first;
    std::vector<uint8_t> host;
    int block = 0;
    if (!p.sdot) {
        p.rot.reserve(size_t(p.count) * p.batch * m.dev);
        std::vector<CqJob> jobs(p.count);
        p.xraw = gemv_prepass(m.group) && gemv_quad_takes_x(m.group, m.in);
        const bool fused = gemv_fuses_fwht(m.group) || p.xraw;
        for (int i = 0; i < p.count; ++i) {
            const Matrix &mi = p.cq[i]->m;
            const float *act = fused ? p.xs_in[i] : p.rot.p + size_t(i) * p.batch * m.dev;
            jobs[i] = CqJob{mi.codes.p, mi.norms.p, act, p.ys[i], mi.out, mi.n_pad, block, p.batch};
            block += mi.n_pad / kRowsPerBlock;
        }
        host.assign(reinterpret_cast<uint8_t *>(jobs.data()), reinterpret_cast<uint8_t *>(jobs.data() + p.count));
        p.xptr.reserve(p.count);
        ND_HIP(hipMemcpy(p.xptr.p, p.xs_in.data(), p.count * sizeof(const float *), hipMemcpyHostToDevice));
    } else {
        p.rot.reserve(size_t(p.count) * p.batch * m.dev);
        p.q.reserve(size_t(p.count) * p.batch * m.dev / 4);
        p.xscale.reserve(size_t(p.count) * p.batch * m.groups);
        p.xscale_t.reserve(size_t(p.count) * p.batch * m.groups);
        std::vector<SdotJob> jobs(p.count);
        // matrices reading one input (a Q|K|V plan) share one prepared copy of it
        const bool shared = std::all_of(p.xs_in.begin(), p.xs_in.end(), [&](const float *x) { return x == p.xs_in[0]; });
        p.inputs = shared ? 1 : p.count;
        for (int i = 0; i < p.count; ++i) {
            const Matrix &mi = p.sd[i]->m;
            const size_t k = shared ? 0 : size_t(i);  // staging slot of matrix i's input
            jobs[i] = SdotJob{mi.codes.p,
                              mi.norms.p,
                              p.q.p + k * p.batch * m.dev / 4,
                              p.xscale.p + k * p.batch * m.groups,
                              p.ys[i],
                              mi.out,
                              mi.n_pad,
                              block,
                              p.batch,
                              p.xscale_t.p + k * p.batch * m.groups,
                              0,
                              p.xs_in[i]};
            block += mi.n_pad / kRowsPerBlock;
        }
        host.assign(reinterpret_cast<uint8_t *>(jobs.data()), reinterpret_cast<uint8_t *>(jobs.data() + p.count));
        p.xptr.reserve(p.count);
        ND_HIP(hipMemcpy(p.xptr.p, p.xs_in.data(), p.count * sizeof(const float *), hipMemcpyHostToDevice));
    }
    p.blocks = block;
    p.jobs.reserve(host.size());
    ND_HIP(hipMemcpy(p.jobs.p, host.data(), host.size(), hipMemcpyHostToDevice));
}

// The int8 plan's input preparation: one launch prepares every (matrix,
// batch row) input into the plan's staging (q, xscale, xscale_t).
static void plan_prepare(Plan &p, hipStream_t s) {
    const Matrix &m = *p.first;
    if (!launch_sdot_prepare(nullptr, p.xptr.p, p.batch, p.inputs * p.batch, m.in, m.padded, m.dev, m.group,
                             m.scale, m.kind, p.q.p, p.xscale.p, p.xscale_t.p, s)) {
        for (int i = 0; i < p.inputs; ++i)
            m.transform(p.xs_in[i], m.in, p.rot.p + size_t(i) * p.batch * m.dev, p.batch, p.st.big, s);
        launch_sdot_quantize(p.rot.p, m.dev, p.inputs * p.batch, m.padded, m.dev, m.group, m.kind, p.q.p,
                             p.xscale.p, s);
    }
}

// Where a producer of `x` (batch rows of n values) may leave `next`'s input
// prepared: next is a one-matrix int8 plan of groups of 32 whose input is
// exactly x. q null otherwise.
PrepOut plan_prep_target(const void *next_plan, const float *x, int n, int batch) {
    PrepOut po{};
    if (!next_plan) return po;
    const Plan &c = *static_cast<const Plan *>(next_plan);
    const Matrix &m = *c.first;
    ND_CHECK(c.sdot && c.count == 1, "chained run: the next plan must be a one-matrix int8 plan");
    ND_CHECK(c.xs_in[0] == x, "chained run: the next plan's input must be this call's output");
    ND_CHECK(m.in == n && c.batch == batch, "chained run: the next plan's input shape differs from this output");
    if (m.group != 32) return po;
    po.q = reinterpret_cast<int8_t *>(c.q.p);
    po.xs = c.xscale.p;
    po.xst = c.xscale_t.p;
    po.dev = m.dev;
    po.padded = m.padded;
    po.groups = m.groups;
    po.kind = m.kind;
    po.batch = c.batch;
    po.scale = m.scale;
    return po;
}

// Whether the int8 plan's GEMV prepares its own input (batch 1, small
// matrices), which then needs no producer to prepare it.
static bool plan_takes_x(const Plan &p) { return p.sdot && sdot_gemv_takes_x(p.sd[0]->geom(), p.blocks, p.batch); }

bool plan_wants_input(const void *next_plan) { return !plan_takes_x(*static_cast<const Plan *>(next_plan)); }

void plan_prepare_input(void *next_plan, hipStream_t s) {
    Plan &c = *static_cast<Plan *>(next_plan);
    plan_prepare(c, s);
    c.staged = true;
}

void plan_mark_staged(void *next_plan) { static_cast<Plan *>(next_plan)->staged = true; }

// prepared: use the prepared input a chained producer call left in the
// staging since this plan's last run (without one, the run prepares its
// input itself). next: an int8 plan whose input is this plan's output, left
// prepared for its run with `prepared` (in the GEMV's epilogue where the
// shapes allow, else by its prepare launch; not at all when next's GEMV
// prepares its own input).
static void plan_run(Plan &p, hipStream_t s, hipEvent_t gemv_start = nullptr, hipEvent_t gemv_stop = nullptr,
                     Plan *next = nullptr, bool prepared = false) {
    const Matrix &m = *p.first;
    ND_CHECK(p.sdot || (!next && !prepared), "chained run: FP32 plans neither take nor leave prepared inputs");
    ND_CHECK(!next || p.count == 1, "chained run: the producing plan must hold one matrix");
    // x_i is [batch][in] on the device; the FP32 GEMV transforms it in-kernel
    // unless the group exceeds one table window
    if (!p.sdot) {
        if (gemv_prepass(m.group) && !p.xraw)
            launch_rot_many(nullptr, p.xptr.p, p.batch, p.count * p.batch, m.in, m.dev, m.group, m.scale, p.rot.p, s);
        else if (!gemv_fuses_fwht(m.group) && !p.xraw)
            for (int i = 0; i < p.count; ++i)
                m.transform(p.xs_in[i], m.in, p.rot.p + size_t(i) * p.batch * m.dev, p.batch, p.st.big, s);
        if (gemv_start) ND_HIP(hipEventRecord(gemv_start, s));
        launch_cq_gemv(m.geom(), CqJob{}, reinterpret_cast<const CqJob *>(p.jobs.p), p.count, p.blocks, s, p.xraw,
                       p.batch);
        if (gemv_stop) ND_HIP(hipEventRecord(gemv_stop, s));
        return;
    }
    const SdotGeom g0 = p.sd[0]->geom();
    const SdotJob *jobs = reinterpret_cast<const SdotJob *>(p.jobs.p);
    const bool staged = prepared && p.staged;
    p.staged = false;
    const PrepOut target = plan_prep_target(next, p.ys[0], m.out, p.batch);  // checks next
    const bool feed = next && plan_wants_input(next);
    const PrepOut po = feed ? target : PrepOut{};
    if (!staged && plan_takes_x(p)) {  // batch 1, small matrices: the GEMV prepares its input
        if (gemv_start) ND_HIP(hipEventRecord(gemv_start, s));
        launch_sdot_gemv_x(g0, SdotJob{}, jobs, p.count, p.blocks, s);
        if (feed) plan_prepare_input(next, s);
    } else {
        if (!staged) plan_prepare(p, s);
        if (gemv_start) ND_HIP(hipEventRecord(gemv_start, s));
        if (launch_sdot_gemv_prep(g0, SdotJob{}, jobs, p.count, p.blocks, p.batch, po, s)) {
            plan_mark_staged(next);
        } else {
            launch_sdot_gemv(g0, SdotJob{}, jobs, p.count, p.blocks, p.batch, s);
            if (feed) plan_prepare_input(next, s);
        }
    }
    if (gemv_stop) ND_HIP(hipEventRecord(gemv_stop, s));
}

static bool same_geometry(const Matrix &a, const Matrix &b) {
    return a.in == b.in && a.bits == b.bits && a.group == b.group && std::memcmp(a.lut, b.lut, sizeof a.lut) == 0;
}

// needle2_cq_linear_many for matrices of one input length and group, staged
// in the first handle's buffers and run on its stream.
static void linear_many(const std::vector<CqHandle *> &hs, const float *x, float *const *ys) {
    CqHandle &h0 = *hs[0];
    const Matrix &m0 = h0.m;
    Staging &st = h0.st;
    const hipStream_t s = st.stream();
    const int n = static_cast<int>(hs.size());
    std::vector<size_t> at(static_cast<size_t>(n) + 1, 0);  // output offsets in the shared y buffer
    for (int i = 0; i < n; ++i) at[i + 1] = at[i] + size_t(hs[i]->m.out);
    st.hx.reserve(m0.in);
    st.x.reserve(m0.in);
    st.y.reserve(at[n]);
    st.hy.reserve(at[n]);
    std::memcpy(st.hx.p, x, size_t(m0.in) * sizeof(float));
    ND_HIP(hipMemcpyAsync(st.x.p, st.hx.p, size_t(m0.in) * sizeof(float), hipMemcpyHostToDevice, s));
    // the one transform: the shared rotated x, unless the GEMV fuses the FWHT into its table build
    const float *act = st.x.p;
    const bool xraw = gemv_prepass(m0.group) && gemv_quad_takes_x(m0.group, m0.in);  // the GEMV transforms x itself
    if (!gemv_fuses_fwht(m0.group) && !xraw) {
        st.rot.reserve(m0.dev);
        if (gemv_prepass(m0.group)) launch_rot_many(st.x.p, nullptr, 1, 1, m0.in, m0.dev, m0.group, m0.scale, st.rot.p, s);
        else m0.transform(st.x.p, m0.in, st.rot.p, 1, st.big, s);
        act = st.rot.p;
    }
    // job tables: one per run of equal storage geometry, all in one upload
    std::vector<CqJob> jobs(static_cast<size_t>(n));
    std::vector<std::pair<int, int>> runs;  // (first job, blocks) per launch
    int block = 0;
    for (int i = 0; i < n; ++i) {
        const Matrix &mi = hs[i]->m;
        if (i == 0 || !same_geometry(mi, hs[runs.back().first]->m)) {
            runs.push_back({i, 0});
            block = 0;
        }
        jobs[i] = CqJob{mi.codes.p, mi.norms.p, act, st.y.p + at[i], mi.out, mi.n_pad, block, 1};
        block += mi.n_pad / kRowsPerBlock;
        runs.back().second = block;
    }
    const size_t table = jobs.size() * sizeof(CqJob);
    st.hjobs.reserve(table);
    st.jobs.reserve(table);
    std::memcpy(st.hjobs.p, jobs.data(), table);
    ND_HIP(hipMemcpyAsync(st.jobs.p, st.hjobs.p, table, hipMemcpyHostToDevice, s));
    for (size_t r = 0; r < runs.size(); ++r) {
        const int first = runs[r].first;
        const int njobs = (r + 1 < runs.size() ? runs[r + 1].first : n) - first;
        launch_cq_gemv(hs[first]->m.geom(), CqJob{}, reinterpret_cast<const CqJob *>(st.jobs.p) + first, njobs,
                       runs[r].second, s, xraw);
    }
    ND_HIP(hipMemcpyAsync(st.hy.p, st.y.p, at[n] * sizeof(float), hipMemcpyDeviceToHost, s));
    ND_HIP(hipStreamSynchronize(s));
    for (int i = 0; i < n; ++i) std::memcpy(ys[i], st.hy.p + at[i], size_t(hs[i]->m.out) * sizeof(float));
}

}  // namespace nd

using namespace nd;

static void poison(float *y, size_t n) {
    if (!y) return;
    const float nan = std::numeric_limits<float>::quiet_NaN();
    for (size_t i = 0; i < n; ++i) y[i] = nan;
}

extern "C" {

// ===================== reference ABI (drop-in) ===========================

const char *needle2_native_features(void) { return "gfx950-hip;float32-accumulate;direct-packed-cq;int8-dot4"; }

void *needle2_cq_create(const uint8_t *p, const uint16_t *n, int out, int in, int bits, int group, const float *cb) {
    CqHandle *h = nullptr;
    int rc = guarded([&] {
        auto u = std::make_unique<CqHandle>();
        u->m.upload(p, n, out, in, bits, group, cb, nullptr);
        h = u.release();
    });
    return rc ? nullptr : h;
}

void needle2_cq_destroy(void *handle) { delete static_cast<CqHandle *>(handle); }

void needle2_cq_linear(void *handle, const float *x, float *y, int batch, int threads) {
    (void)threads;
    auto *h = static_cast<CqHandle *>(handle);
    if (guarded([&] { h->linear_host(x, y, batch); })) poison(y, size_t(batch > 0 ? batch : 0) * h->m.out);
}

// The reference's activation-table modes 1-3 are alternative CPU summation
// schemes with the same tolerance contract (tests/test_native.py:39-40); on
// the GPU every mode runs the packed GEMV.
void needle2_cq_linear_lookup(void *handle, const float *x, float *y, int batch, int threads, int mode) {
    (void)mode;
    needle2_cq_linear(handle, x, y, batch, threads);
}

// cq.cpp:287-292, 360-366: one x through several matrices. When every
// matrix takes the same input length and group (the reference's
// compatible_rotation), x is copied in once and transformed once, and each
// run of matrices with one storage geometry (bits and codebook) is one GEMV
// launch over a job table; all outputs come back in one copy and one wait.
// Otherwise each matrix runs on its own, as the reference falls back. Every
// mode runs the same GEMV (the reference's table modes are other CPU
// summation orders under one tolerance contract).
void needle2_cq_linear_many(void *const *handles, int count, const float *x, float *const *ys, int threads, int mode) {
    (void)threads;
    (void)mode;
    if (count <= 0) return;
    std::vector<CqHandle *> hs(static_cast<size_t>(count));
    for (int i = 0; i < count; ++i) hs[i] = static_cast<CqHandle *>(handles[i]);
    bool shared = true;
    for (int i = 1; i < count; ++i) shared = shared && hs[i]->m.in == hs[0]->m.in && hs[i]->m.group == hs[0]->m.group;
    const int rc = guarded([&] {
        if (!shared) {
            for (int i = 0; i < count; ++i) hs[i]->linear_host(x, ys[i], 1);
            return;
        }
        linear_many(hs, x, ys);
    });
    if (rc)
        for (int i = 0; i < count; ++i) poison(ys[i], size_t(hs[i]->m.out));
}

void needle2_cq_rows(void *handle, const int64_t *ids, float *y, int count) {
    auto *h = static_cast<CqHandle *>(handle);
    if (guarded([&] { h->rows_host(ids, y, count); })) poison(y, size_t(count > 0 ? count : 0) * h->m.in);
}

int needle2_sdot_supported(void) { return 1; }

static void *sdot_create_impl(const uint8_t *p, const uint16_t *n, int out, int in, int bits, int group,
                              const float *cb, int min_group, hipStream_t stream = nullptr,
                              bool device_inputs = false) {
    SdotHandle *h = nullptr;
    int rc = guarded([&] {
        ND_CHECK(bits == 2 || bits == 4, "SDOT requires CQ2/CQ4");
        ND_CHECK(group >= min_group && group <= 131072, "SDOT group size outside the supported range");
        ND_CHECK(bits == 4 || group >= 16, "SDOT CQ2 requires group >= 16");
        auto u = std::make_unique<SdotHandle>();
        u->m.upload(p, n, out, in, bits, group, cb, stream, device_inputs);
        u->init_tables();
        h = u.release();
    });
    return rc ? nullptr : h;
}

// sdot.cpp:351-354: bits in {2,4}, group in [64, 131072].
void *needle2_sdot_create(const uint8_t *p, const uint16_t *n, int out, int in, int bits, int group, const float *cb) {
    return sdot_create_impl(p, n, out, in, bits, group, cb, 64);
}

void needle2_sdot_destroy(void *p) { delete static_cast<SdotHandle *>(p); }

void needle2_sdot_linear(void *p, const float *x, float *y, int batch, int threads) {
    (void)threads;
    auto *h = static_cast<SdotHandle *>(p);
    if (guarded([&] { h->linear_host(x, y, batch); })) poison(y, size_t(batch > 0 ? batch : 0) * h->m.out);
}

// ===================== additive gfx950 exports ===========================

const char *needle2_gpu_error(void) { return get_error(); }

// Same arithmetic as needle2_sdot_create, with groups down to 8 (CQ4) / 16 (CQ2).
void *needle2_gpu_sdot_create(const uint8_t *p, const uint16_t *n, int out, int in, int bits, int group,
                              const float *cb) {
    return sdot_create_impl(p, n, out, in, bits, group, cb, 8);
}

// Creation from device-resident packed codes and norms (the reference's
// layouts): the relayout kernels are enqueued on `stream` and the call returns
// without waiting, so a whole model's matrices can be built from one bulk copy
// of its archive; the inputs must stay valid until the stream has run them.
void *needle2_gpu_cq_create_device(const uint8_t *d_packed, const uint16_t *d_norms, int out, int in, int bits,
                                   int group, const float *cb, void *stream) {
    CqHandle *h = nullptr;
    int rc = guarded([&] {
        auto u = std::make_unique<CqHandle>();
        u->m.upload(d_packed, d_norms, out, in, bits, group, cb, static_cast<hipStream_t>(stream), true);
        h = u.release();
    });
    return rc ? nullptr : h;
}

void *needle2_gpu_sdot_create_device(const uint8_t *d_packed, const uint16_t *d_norms, int out, int in, int bits,
                                     int group, const float *cb, void *stream) {
    return sdot_create_impl(d_packed, d_norms, out, in, bits, group, cb, 8, static_cast<hipStream_t>(stream), true);
}

int needle2_gpu_cq_linear_device(void *handle, const float *d_x, float *d_y, int batch, void *stream) {
    auto *h = static_cast<CqHandle *>(handle);
    return guarded([&] { h->run_device(d_x, d_y, batch, stream ? static_cast<hipStream_t>(stream) : h->st.stream()); });
}

// Prefill GEMM: d_y[m][out] = d_x[m][in] through the matrix on fp16 MFMA
// (fp32 accumulation); the batched form of needle2_cq_linear used for prompt
// chunks (engine.cpp:607-670). 4-bit codes (CQ4, CQ3).
int needle2_gpu_cq_gemm_device(void *handle, const float *d_x, float *d_y, int m, void *stream) {
    return guarded([&] {
        ND_CHECK(handle, "null CQ handle");
        auto *h = static_cast<CqHandle *>(handle);
        h->gemm_device(d_x, d_y, m, stream ? static_cast<hipStream_t>(stream) : h->st.stream(), nullptr, nullptr);
    });
}

// As needle2_gpu_cq_gemm_device, with two events recorded around `repeat`
// back-to-back launches of the GEMM kernel (after one activation transform):
// the per-launch time is the elapsed time / repeat.
int needle2_gpu_cq_gemm_timed(void *handle, const float *d_x, float *d_y, int m, void *stream, void *gemm_start,
                              void *gemm_stop, int repeat) {
    return guarded([&] {
        ND_CHECK(handle, "null CQ handle");
        ND_CHECK(repeat >= 1, "repeat must be >= 1");
        auto *h = static_cast<CqHandle *>(handle);
        h->gemm_device(d_x, d_y, m, stream ? static_cast<hipStream_t>(stream) : h->st.stream(),
                       static_cast<hipEvent_t>(gemm_start), static_cast<hipEvent_t>(gemm_stop), repeat);
    });
}

int needle2_gpu_sdot_linear_device(void *handle, const float *d_x, float *d_y, int batch, void *stream) {
    auto *h = static_cast<SdotHandle *>(handle);
    return guarded([&] { h->run_device(d_x, d_y, batch, stream ? static_cast<hipStream_t>(stream) : h->st.stream()); });
}

// The int32 group dots of the int8 product (sdot.cpp:108-137): d_dots[b][row][g],
// from the kernels the GEMV runs for this batch on a large matrix.
int needle2_gpu_sdot_dots_device(void *handle, const float *d_x, int32_t *d_dots, int batch, void *stream) {
    return guarded([&] {
        ND_CHECK(handle && d_x && d_dots, "int8 dots: null argument");
        auto *h = static_cast<SdotHandle *>(handle);
        h->dots_device(d_x, d_dots, batch, stream ? static_cast<hipStream_t>(stream) : h->st.stream());
    });
}

// Candidate rows: y[i] = row ids[i] of the product for one input vector, as
// Engine::project_candidates computes them (engine.cpp:1302-1349; ids must be
// nonempty and inside [0, out): -1 with the reference's messages otherwise).
int needle2_gpu_cq_candidates(void *handle, const float *x, const int32_t *ids, int count, float *y) {
    return guarded([&] {
        ND_CHECK(handle && x && y, "null argument");
        static_cast<CqHandle *>(handle)->candidates_host(x, ids, count, y);
    });
}

int needle2_gpu_cq_candidates_device(void *handle, const float *d_x, const int32_t *d_ids, int count, float *d_y,
                                     void *stream) {
    return guarded([&] {
        ND_CHECK(handle, "null CQ handle");
        ND_CHECK(count > 0, "candidates must be nonempty");
        auto *h = static_cast<CqHandle *>(handle);
        h->candidates_device(d_x, d_ids, count, d_y, stream ? static_cast<hipStream_t>(stream) : h->st.stream());
    });
}

int needle2_gpu_sdot_candidates(void *handle, const float *x, const int32_t *ids, int count, float *y) {
    return guarded([&] {
        ND_CHECK(handle && x && y, "null argument");
        static_cast<SdotHandle *>(handle)->candidates_host(x, ids, count, y);
    });
}

int needle2_gpu_sdot_candidates_device(void *handle, const float *d_x, const int32_t *d_ids, int count, float *d_y,
                                       void *stream) {
    return guarded([&] {
        ND_CHECK(handle, "null SDOT handle");
        ND_CHECK(count > 0, "candidates must be nonempty");
        auto *h = static_cast<SdotHandle *>(handle);
        h->candidates_device(d_x, d_ids, count, d_y, stream ? static_cast<hipStream_t>(stream) : h->st.stream());
    });
}

// Plans: count matrices sharing (in, bits, group, codebook); matrix i reads
// d_x[i] ([batch][in], device) and writes d_y[i] ([batch][out_i], device).
static void *plan_create(void *const *handles, int count, const float *const *d_x, float *const *d_y, int batch,
                         bool sdot) {
    Plan *out = nullptr;
    guarded([&] {
        ND_CHECK(count > 0 && batch > 0, "plan needs matrices and batch >= 1");
        auto p = std::make_unique<Plan>();
        p->sdot = sdot;
        p->count = count;
        p->batch = batch;
        for (int i = 0; i < count; ++i) {
            if (sdot) p->sd.push_back(static_cast<SdotHandle *>(handles[i]));
            else p->cq.push_back(static_cast<CqHandle *>(handles[i]));
            p->xs_in.push_back(d_x[i]);
            p->ys.push_back(d_y[i]);
        }
        p->first = sdot ? &p->sd[0]->m : &p->cq[0]->m;
        for (int i = 1; i < count; ++i)
            ND_CHECK(same_geometry(*p->first, sdot ? p->sd[i]->m : p->cq[i]->m),
                     "plan matrices must share input size, bits, group and codebook");
        plan_upload(*p);
        out = p.release();
    });
    return out;
}

void *needle2_gpu_cq_plan_create(void *const *handles, int count, const float *const *d_x, float *const *d_y,
                                 int batch) {
    return plan_create(handles, count, d_x, d_y, batch, false);
}

void *needle2_gpu_sdot_plan_create(void *const *handles, int count, const float *const *d_x, float *const *d_y,
                                   int batch) {
    return plan_create(handles, count, d_x, d_y, batch, true);
}

int needle2_gpu_plan_run(void *plan, void *stream) {
    auto *p = static_cast<Plan *>(plan);
    return guarded([&] { plan_run(*p, stream ? static_cast<hipStream_t>(stream) : p->st.stream()); });
}

// As needle2_gpu_plan_run, also recording two events on the stream right
// before and right after the GEMV launch (the plan's dominant kernel).
int needle2_gpu_plan_run_timed(void *plan, void *stream, void *gemv_start, void *gemv_stop) {
    auto *p = static_cast<Plan *>(plan);
    return guarded([&] {
        plan_run(*p, stream ? static_cast<hipStream_t>(stream) : p->st.stream(), static_cast<hipEvent_t>(gemv_start),
                 static_cast<hipEvent_t>(gemv_stop));
    });
}

// A run in a chain of int8 plans (a decode layer's O -> MLP up -> MLP down):
// with `prepared` non-zero the plan uses the prepared input that a chained
// call of its producer (this call or needle2_gpu_attention_chained with
// `next` = this plan) left in its staging since its last run, and prepares
// its input itself when none did; with `next` not NULL (a one-matrix int8
// plan whose input buffer is this plan's output) the run also leaves next's
// input prepared, for next's run with `prepared`. Outputs are the bits of
// unchained runs. The calls of one chain go to one stream, in order.
int needle2_gpu_plan_run_chained(void *plan, void *next, int prepared, void *stream) {
    auto *p = static_cast<Plan *>(plan);
    return guarded([&] {
        plan_run(*p, stream ? static_cast<hipStream_t>(stream) : p->st.stream(), nullptr, nullptr,
                 static_cast<Plan *>(next), prepared != 0);
    });
}

void needle2_gpu_plan_destroy(void *plan) { delete static_cast<Plan *>(plan); }

// ---- memory, streams, events -------------------------------------------
void *needle2_gpu_malloc(size_t bytes) {
    void *p = nullptr;
    if (guarded([&] { ND_HIP(hipMalloc(&p, bytes ? bytes : 1)); })) return nullptr;
    return p;
}

void needle2_gpu_free(void *p) {
    if (p) (void)hipFree(p);
}

// kind: 0 host->device, 1 device->host, 2 device->device
int needle2_gpu_memcpy(void *dst, const void *src, size_t bytes, int kind) {
    return guarded([&] {
        hipMemcpyKind k = kind == 0 ? hipMemcpyHostToDevice : kind == 1 ? hipMemcpyDeviceToHost : hipMemcpyDeviceToDevice;
        ND_HIP(hipMemcpy(dst, src, bytes, k));
    });
}

// Streaming device-to-device copy kernel (bytes rounded down to 16).
int needle2_gpu_copy_kernel(void *dst, const void *src, size_t bytes, void *stream) {
    return guarded([&] { launch_copy(src, dst, bytes, static_cast<hipStream_t>(stream)); });
}

// Calibration of the limits the kernels are measured against (no
// counterpart in the reference).
int needle2_gpu_calib_launch(int launches, float *us_per_launch, void *stream) {
    return guarded([&] {
        ND_CHECK(launches > 0 && us_per_launch, "launch calibration: launches > 0 and an output");
        *us_per_launch = calib_launch_us(launches, static_cast<hipStream_t>(stream));
    });
}

int needle2_gpu_calib_lds(int width, float *bytes_per_clk_per_cu, float *shader_ghz, void *stream) {
    return guarded([&] {
        ND_CHECK(width == 4 || width == 8 || width == 16, "LDS calibration: width 4, 8 or 16 bytes");
        ND_CHECK(bytes_per_clk_per_cu && shader_ghz, "LDS calibration: null output");
        calib_lds(width, bytes_per_clk_per_cu, shader_ghz, static_cast<hipStream_t>(stream));
    });
}

int needle2_gpu_calib_stream(const void *d_src, size_t bytes, int pattern, float *us, void *stream) {
    return guarded([&] {
        ND_CHECK(d_src && us && pattern >= 0 && pattern <= 3, "stream calibration: buffer, output, pattern 0-3");
        *us = calib_stream_us(d_src, bytes, pattern, static_cast<hipStream_t>(stream));
    });
}

int needle2_gpu_memset(void *dst, int value, size_t bytes) {
    return guarded([&] { ND_HIP(hipMemset(dst, value, bytes)); });
}

int needle2_gpu_synchronize(void) {
    return guarded([&] { ND_HIP(hipDeviceSynchronize()); });
}

void *needle2_gpu_stream_create(void) {
    hipStream_t s = nullptr;
    if (guarded([&] { ND_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)); })) return nullptr;
    return s;
}

void needle2_gpu_stream_destroy(void *s) {
    if (s) (void)hipStreamDestroy(static_cast<hipStream_t>(s));
}

int needle2_gpu_stream_synchronize(void *s) {
    return guarded([&] { ND_HIP(hipStreamSynchronize(static_cast<hipStream_t>(s))); });
}

// HIP graphs: capture the work issued to `stream` between begin and end
// (thread-local capture mode), instantiate it, and replay it with one launch.
// Only launches belong in a capture: every entry point used inside must have
// run once before (their grow-only buffers are then allocated) and must not
// copy from host memory or wait on the host.
int needle2_gpu_graph_begin(void *stream) {
    return guarded([&] {
        ND_CHECK(stream, "graph capture needs a stream created by needle2_gpu_stream_create");
        ND_HIP(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal));
    });
}

void *needle2_gpu_graph_end(void *stream) {
    hipGraphExec_t exec = nullptr;
    if (guarded([&] {
            hipGraph_t graph = nullptr;
            ND_HIP(hipStreamEndCapture(static_cast<hipStream_t>(stream), &graph));
            const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            ND_HIP(e);
        }))
        return nullptr;
    return exec;
}

int needle2_gpu_graph_launch(void *graph, void *stream) {
    return guarded([&] {
        ND_CHECK(graph, "graph launch: null graph");
        ND_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), static_cast<hipStream_t>(stream)));
    });
}

void needle2_gpu_graph_destroy(void *graph) {
    if (graph) (void)hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph));
}

// Timing events: no system-scope fence when recorded (no L2 write-back and
// invalidate between the kernels being timed), so an event pair brackets the
// kernel itself. needle2_gpu_event_elapsed still waits for the stop event.
void *needle2_gpu_event_create(void) {
    hipEvent_t e = nullptr;
    if (guarded([&] { ND_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence)); })) return nullptr;
    return e;
}

void needle2_gpu_event_destroy(void *e) {
    if (e) (void)hipEventDestroy(static_cast<hipEvent_t>(e));
}

int needle2_gpu_event_record(void *e, void *s) {
    return guarded([&] { ND_HIP(hipEventRecord(static_cast<hipEvent_t>(e), static_cast<hipStream_t>(s))); });
}

// milliseconds between two recorded events (waits for the second)
float needle2_gpu_event_elapsed(void *start, void *stop) {
    float ms = -1.0f;
    guarded([&] {
        ND_HIP(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
        ND_HIP(hipEventElapsedTime(&ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
    });
    return ms;
}

// "name;gfx;cus;hbm_bytes;clock_khz"
int needle2_gpu_device_info(char *buf, int len) {
    return guarded([&] {
        int dev = 0;
        ND_HIP(hipGetDevice(&dev));
        hipDeviceProp_t prop;
        ND_HIP(hipGetDeviceProperties(&prop, dev));
        std::string s = std::string(prop.name) + ";" + prop.gcnArchName + ";" + std::to_string(prop.multiProcessorCount) +
                        ";" + std::to_string(prop.totalGlobalMem) + ";" + std::to_string(prop.clockRate);
        std::snprintf(buf, size_t(len), "%s", s.c_str());
    });
}

}  // extern "C"
