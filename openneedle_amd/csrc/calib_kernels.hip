// Hardware calibration kernels: the measured limits the GEMV, attention and
// decode-layer kernels are compared against (dependent launch latency, LDS
// read rate by access width, HBM streaming rate of the GEMVs' per-tile walk
// with plain and non-temporal loads). Not on any compute path.
#include "common.h"

namespace nd {

namespace {

__global__ void empty_kernel() {}

// LDS read rate: every lane reads its own column (lane * W bytes) of 16 rows
// of 64 * W bytes per iteration, with immediate offsets (no address VALU);
// the row set alternates so the reads cannot be hoisted. Wave 0 of block 0
// records s_memtime and s_memrealtime (100 MHz) around its loop, giving the
// shader clock of the run.
constexpr int kLdsProbeBytes = 32768, kLdsProbeIter = 256;

template <int W>
__global__ __launch_bounds__(256) void lds_probe_kernel(uint32_t *out, uint64_t *clk) {
    __shared__ __attribute__((aligned(16))) uint32_t t[kLdsProbeBytes / 4];
    for (int i = threadIdx.x; i < kLdsProbeBytes / 4; i += 256) t[i] = i * 2654435761u;
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const uint64_t c0 = __builtin_readcyclecounter(), r0 = __builtin_amdgcn_s_memrealtime();
    uint32_t acc = 0;
    for (int it = 0; it < kLdsProbeIter; ++it) {
        uint32_t off = lane * W + (it & 1) * (16 * 64 * W);  // < 32 * 64 * 16 = 32 KiB
        asm volatile("" : "+v"(off));
        const char *b = reinterpret_cast<const char *>(t) + off;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const char *p = b + e * (64 * W);
            if constexpr (W == 4) {
                acc += *reinterpret_cast<const uint32_t *>(p);
            } else if constexpr (W == 8) {
                const uint2 v = *reinterpret_cast<const uint2 *>(p);
                acc += v.x ^ v.y;
            } else {
                const u32x4 v = *reinterpret_cast<const u32x4 *>(p);
                acc += v.x ^ v.y ^ v.z ^ v.w;
            }
        }
    }
    const uint64_t c1 = __builtin_readcyclecounter(), r1 = __builtin_amdgcn_s_memrealtime();
    out[blockIdx.x * 256 + threadIdx.x] = acc;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        clk[0] = c1 - c0;
        clk[1] = r1 - r0;
    }
}

// The GEMVs' HBM walk: one 1024-thread workgroup per tile of `tile` bytes
// (16-byte pieces, one per thread per 16 KiB step, three steps in flight),
// each tile read front to back, with plain (AUX 0) or non-temporal loads.
template <int AUX>
__global__ __launch_bounds__(1024) void tile_walk_kernel(const uint8_t *__restrict__ src, uint32_t tile,
                                                         uint32_t *out) {
    const auto r = buffer_rsrc(src + static_cast<size_t>(blockIdx.x) * tile, tile);
    const uint32_t lane16 = threadIdx.x * 16u, steps = tile / (1024u * 16u);
    u32x4 v[3];
    uint32_t acc = 0;
    v[0] = __builtin_amdgcn_raw_buffer_load_b128(r, lane16, 0, AUX);
    v[1] = __builtin_amdgcn_raw_buffer_load_b128(r, lane16, 16384, AUX);
    for (uint32_t s = 0; s < steps; s += 3) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            // step s + k + 2 (past the tile: reads zero through the buffer bound)
            v[(k + 2) % 3] = __builtin_amdgcn_raw_buffer_load_b128(r, lane16, (s + k + 2) * 16384u, AUX);
            acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
        }
    }
    out[blockIdx.x * 1024 + threadIdx.x] = acc;
}

// Plain grid-stride streaming, 16 bytes per lane per step.
template <bool NT>
__global__ __launch_bounds__(256) void grid_stream_kernel(const u32x4 *__restrict__ src, size_t n, uint32_t *out) {
    uint32_t acc = 0;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<size_t>(gridDim.x) * 256) {
        const u32x4 v = NT ? __builtin_nontemporal_load(src + i) : src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    out[blockIdx.x * 256 + threadIdx.x] = acc;
}

// Mean milliseconds per call of `launch` over `reps` calls on stream s,
// between fence-free timing events, after `warm` untimed calls.
template <class F>
float timed_ms(F &&launch, int warm, int reps, hipStream_t s) {
    for (int i = 0; i < warm; ++i) launch();
    hipEvent_t a = nullptr, b = nullptr;
    ND_HIP(hipEventCreateWithFlags(&a, hipEventDisableSystemFence));
    ND_HIP(hipEventCreateWithFlags(&b, hipEventDisableSystemFence));
    ND_HIP(hipEventRecord(a, s));
    for (int i = 0; i < reps; ++i) launch();
    ND_HIP(hipEventRecord(b, s));
    ND_HIP(hipEventSynchronize(b));
    float ms = 0.0f;
    ND_HIP(hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    ND_HIP(hipGetLastError());
    return ms / static_cast<float>(reps);
}

}  // namespace

float calib_launch_us(int launches, hipStream_t s) {
    return 1e3f * timed_ms([&] { hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, s); }, 20, launches, s);
}

void calib_lds(int width, float *bytes_per_clk_per_cu, float *ghz, hipStream_t s) {
    int dev = 0, cus = 256;
    ND_HIP(hipGetDevice(&dev));
    ND_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int blocks = cus * 16;  // 32 KiB of LDS per block: 4 blocks (16 waves) per CU, several rounds
    DevBuf<uint32_t> out;
    DevBuf<uint64_t> clk;
    out.reserve(static_cast<size_t>(blocks) * 256);
    clk.reserve(2);
    auto go = [&] {
        switch (width) {
        case 4: hipLaunchKernelGGL(lds_probe_kernel<4>, dim3(blocks), dim3(256), 0, s, out.p, clk.p); break;
        case 8: hipLaunchKernelGGL(lds_probe_kernel<8>, dim3(blocks), dim3(256), 0, s, out.p, clk.p); break;
        default: hipLaunchKernelGGL(lds_probe_kernel<16>, dim3(blocks), dim3(256), 0, s, out.p, clk.p); break;
        }
    };
    const float ms = timed_ms(go, 3, 20, s);
    uint64_t h[2] = {0, 0};
    ND_HIP(hipMemcpy(h, clk.p, sizeof h, hipMemcpyDeviceToHost));
    const double clock_ghz = h[1] ? static_cast<double>(h[0]) / (static_cast<double>(h[1]) / 100e6) / 1e9 : 0.0;
    const double bytes = static_cast<double>(blocks) * 256 * kLdsProbeIter * 16 * width;
    const double per_cu_per_ns = bytes / (ms * 1e6) / cus;
    *ghz = static_cast<float>(clock_ghz);
    *bytes_per_clk_per_cu = clock_ghz > 0 ? static_cast<float>(per_cu_per_ns / clock_ghz) : 0.0f;
}

float calib_stream_us(const void *src, size_t bytes, int pattern, hipStream_t s) {
    // three regions of bytes / 3, read in turn, so no pass finds the previous one in the last-level cache
    const size_t region = bytes / 3 / 16 * 16;
    DevBuf<uint32_t> out;
    int rep = 0;
    if (pattern <= 1) {
        const uint32_t tile = static_cast<uint32_t>(region / 512 / (3 * 16384) * (3 * 16384));  // whole 3-step rounds
        ND_CHECK(tile >= 3 * 16384, "stream calibration: buffer too small");
        out.reserve(512 * 1024);
        return 1e3f * timed_ms([&] {
            const auto *p = static_cast<const uint8_t *>(src) + (rep++ % 3) * region;
            if (pattern == 1) hipLaunchKernelGGL(tile_walk_kernel<kStreamLoad>, dim3(512), dim3(1024), 0, s, p, tile, out.p);
            else hipLaunchKernelGGL(tile_walk_kernel<0>, dim3(512), dim3(1024), 0, s, p, tile, out.p);
        }, 6, 30, s);
    }
    const int grid = 2048;
    out.reserve(static_cast<size_t>(grid) * 256);
    return 1e3f * timed_ms([&] {
        const auto *p = reinterpret_cast<const u32x4 *>(static_cast<const uint8_t *>(src) + (rep++ % 3) * region);
        if (pattern == 3) hipLaunchKernelGGL(grid_stream_kernel<true>, dim3(grid), dim3(256), 0, s, p, region / 16, out.p);
        else hipLaunchKernelGGL(grid_stream_kernel<false>, dim3(grid), dim3(256), 0, s, p, region / 16, out.p);
    }, 6, 30, s);
}

}  // namespace nd
