// int8 GEMV on device buffers without any allocation.
//
// needle2_gpu_sdot_linear_device grows per-handle staging buffers with
// hipMalloc on first use (the quantized activations and their scales). Code
// that must not allocate (work captured into a HIP graph, a serving loop
// that forbids allocation after warm-up) calls
// needle2_gpu_sdot_linear_device_noalloc instead: the same prepare and GEMV
// kernels, with that staging carved out of one file-scope device array,
// `scratch`, which every GPU the library runs on holds until the process
// ends.
//
// The array's name is only a host-side stand-in: its device address, per
// device, comes from hipGetSymbolAddress, called once per device with that
// device current (on the first call made on it) and kept in g_scratch. Every
// use below goes through that address.
//
// Nothing in the scratch has to start at zero: the prepare kernel writes
// every activation byte (all device positions of every batch row) and every
// group scale the GEMV then reads. All calls on one GPU share its array, so
// calls that overlap in time on one GPU (different streams, different host
// threads) race and must be serialized by the caller.
#include "abi_internal.h"

#include <mutex>

namespace nd {
namespace {

constexpr size_t kScratchBytes = size_t(4) << 20;  // per GPU
constexpr size_t kScratchAlign = 256;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
uint8_t *g_scratch[kMaxDevices] = {};
hipError_t g_lookup[kMaxDevices] = {};

// The device address of `scratch` on the current device (looked up once per device).
uint8_t *scratch_address() {
    int dev = 0;
    ND_HIP(hipGetDevice(&dev));
    ND_CHECK(dev >= 0 && dev < kMaxDevices, "no-alloc entry point: device index out of range");
    std::call_once(g_once[dev], [dev] {
        void *p = nullptr;
        g_lookup[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch[dev] = static_cast<uint8_t *>(p);
    });
    ND_HIP(g_lookup[dev]);
    ND_CHECK(g_scratch[dev] != nullptr, "no-alloc entry point: scratch symbol has no device address");
    return g_scratch[dev];
}

size_t aligned(size_t bytes) { return (bytes + kScratchAlign - 1) / kScratchAlign * kScratchAlign; }

}  // namespace
}  // namespace nd

using namespace nd;

extern "C" {

// needle2_gpu_sdot_linear_device with its staging in the library's static
// scratch: d_x [batch][in] and d_y [batch][out] on the device, enqueued on
// `stream` (NULL: the null stream). Refused (-1) when
// batch * (P + 8 * groups) bytes exceed 4 MiB, P being the input padded to
// whole groups and then to a multiple of 256 (the device row, m.dev), each
// of the two parts rounded up to 256 bytes, or when the group is above the
// fused prepare's limit.
int needle2_gpu_sdot_linear_device_noalloc(void *sdot_handle, const float *d_x, float *d_y, int batch,
                                           void *stream) {
    return guarded([&] {
        ND_CHECK(sdot_handle, "null int8 handle");
        if (batch <= 0) return;
        ND_CHECK(d_x && d_y, "no-alloc int8 GEMV: null input or output");
        auto *h = static_cast<SdotHandle *>(sdot_handle);
        const Matrix &m = h->m;
        ND_CHECK(m.group <= kSdotFusedPrepareMaxGroup,
                 "no-alloc int8 GEMV: groups above 16384 need the two-pass prepare; use needle2_gpu_sdot_linear_device");
        const size_t q_bytes = aligned(size_t(batch) * m.dev);
        const size_t s_bytes = aligned(size_t(batch) * m.groups * sizeof(float));
        ND_CHECK(q_bytes + 2 * s_bytes <= kScratchBytes,
                 "no-alloc int8 GEMV: batch * (input padded to whole groups, then to a multiple of 256, + 8 * groups) "
                 "bytes exceed the 4 MiB scratch");
        uint8_t *base = scratch_address();
        auto *q = reinterpret_cast<int32_t *>(base);
        auto *xs = reinterpret_cast<float *>(base + q_bytes);
        auto *xst = reinterpret_cast<float *>(base + q_bytes + s_bytes);
        const hipStream_t s = static_cast<hipStream_t>(stream);
        ND_CHECK(launch_sdot_prepare(d_x, nullptr, batch, batch, m.in, m.padded, m.dev, m.group, m.scale, m.kind, q,
                                     xs, xst, s),
                 "no-alloc int8 GEMV: fused prepare refused the group");
        const SdotJob job{m.codes.p, m.norms.p, q, xs, d_y, m.out, m.n_pad, 0, batch, xst};
        launch_sdot_gemv(h->geom(), job, nullptr, 0, m.n_pad / kRowsPerBlock, batch, s);
    });
}

}  // extern "C"
