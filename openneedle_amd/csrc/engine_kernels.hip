// Glue kernels of the single-sequence engine (needle2/csrc/engine.cpp:968-1044
// for one token, 1045-1301 for a prompt chunk, and the helpers they call).
// The glue kernels run one workgroup per token (blockIdx.y; the attention
// one per kv head, plus the routing workgroup) over the model's small
// vectors (d_model, the mHC lanes, one token's heads), in the reference's
// formulas and operation order per element; block-wide sums and maxima are
// tree reductions, so results agree
// with the reference to fp32 rounding rather than bit for bit. A token's
// arithmetic does not depend on how many tokens share the launch.
//   rms(x, gain)        y = x * (1 / sqrt(sum(x^2) / n + 1e-6)) * (1 + gain)   (engine.cpp:181-184)
//   activation_quant    x = clamp(rint(x / (a / m)), -m-1, m) * (a / m), a = max|x|, m = 2^(bits-1)-1
//   sigmoid(x)          1 / (1 + exp(-x))
//   hadamard(v, n)      butterflies h = 1, 2, .., n/2 of (a + b, a - b), then * 1/sqrt(n)   (cq.cpp:30-46)
//   sinkhorn(a, n)      20 row / column normalisations after exp(a - max)     (engine.cpp:151-180)
#include "engine.h"
#include "sdot_prepare.h"
#include "wave.h"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace nd {

namespace {

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// Four int8 codes (little-endian bytes of w) as floats.
__device__ __forceinline__ float4 int8x4_to_float4(uint32_t w) {
    return make_float4(static_cast<float>(static_cast<int8_t>(w & 0xFFu)),
                       static_cast<float>(static_cast<int8_t>((w >> 8) & 0xFFu)),
                       static_cast<float>(static_cast<int8_t>((w >> 16) & 0xFFu)),
                       static_cast<float>(static_cast<int8_t>(w >> 24)));
}

// Token t's vectors (EngineBufs documents the per-token sizes).
__device__ __forceinline__ EngineBufs at_token(EngineBufs b, const EngineDims &d, int t) {
    const size_t nd = static_cast<size_t>(d.N) * d.D;
    b.x += t * nd;
    b.nx += t * nd;
    b.u += t * d.D;
    b.bx += t * d.D;
    b.z += t * d.D;
    b.proj += t * d.D;
    b.oparts += static_cast<size_t>(t) * d.KV * d.D;
    b.e += t * d.D;
    b.rawv += t * d.D;
    b.zf += t * d.D;
    b.q += t * d.A;
    b.gate += t * d.A;
    b.att += t * d.A;
    b.k += t * d.K;
    b.v += t * d.K;
    b.hidden += static_cast<size_t>(t) * d.layers * d.D;
    b.hpre += t * d.N;
    b.hpost += t * d.N;
    b.hres += t * d.N * d.N;
    b.hroute += t * d.N * d.N;
    for (int m = 0; m < 3; ++m) b.mhc_out[m] += t * d.mhc_stride;
    b.ek += t * d.sites * d.D;
    b.ev += t * d.sites * d.D;
    b.slots += static_cast<size_t>(t) * d.capacity;
    return b;
}

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// p[i] for 0 <= i < n, else 0: a buffer load, so a thread past the end takes
// no branch (a conditional load whose result merges with a default can make
// the compiler wait for the load right away).
__device__ __forceinline__ float load_or_zero(const float *p, int n, int i) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(p, static_cast<uint32_t>(n) * 4u),
                                                                          static_cast<uint32_t>(i) * 4u, 0, 0));
}

// Reads one dword of every 64-byte line of the first BYTES bytes of the
// kernel's arguments, all in one round of scalar loads. The compiler otherwise
// loads argument fields where they are used, and a field indexed at run time
// (or used late) costs a dependent round trip to memory at the kernel's start
// for each line not yet in the scalar cache; after this they hit it.
template <size_t BYTES>
__device__ __forceinline__ void touch_kernargs() {
    typedef const __attribute__((address_space(4))) uint32_t karg_t;
    karg_t *k = (karg_t *)__builtin_amdgcn_kernarg_segment_ptr();
    constexpr int kLines = (BYTES + 63) / 64;
    static_assert(kLines <= 16, "arguments of at most 16 lines");
    uint32_t v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = i < kLines ? k[16 * i] : 0u;
    // one statement uses every value, so every load is in flight before the first wait
    asm volatile("" ::"s"(v[0]), "s"(v[1]), "s"(v[2]), "s"(v[3]), "s"(v[4]), "s"(v[5]), "s"(v[6]), "s"(v[7]),
                 "s"(v[8]), "s"(v[9]), "s"(v[10]), "s"(v[11]), "s"(v[12]), "s"(v[13]), "s"(v[14]), "s"(v[15]));
}

// Block-wide sum / max of one value per thread (every thread gets the result).
__device__ float block_sum(float v, float *red) {
    v = wave_sum(v, threadIdx.x & 63);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) s += red[w];
    return s;
}

// block_sum without its first barrier, for calls that alternate between two
// red buffers: the barrier inside the call between two uses of one buffer
// orders the earlier call's reads before the later call's writes.
__device__ float block_sum_nb(float v, float *red) {
    v = wave_sum(v, threadIdx.x & 63);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) s += red[w];
    return s;
}

__device__ float block_max(float v, float *red) {
    v = wave_max(v, threadIdx.x & 63);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) m = fmaxf(m, red[w]);
    return m;
}

// y = rms(x) (* (1 + gain)); x and y may alias. Ends with a barrier.
__device__ void rms_block(const float *x, float *y, int n, const float *gain, float *red) {
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s += x[i] * x[i];
    s = block_sum(s, red);
    const float r = 1.0f / sqrtf(s / static_cast<float>(n) + 1e-6f);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = x[i] * r;
        y[i] = gain ? v * (1.0f + gain[i]) : v;
    }
    __syncthreads();
}

// engine.cpp:185-190. Ends with a barrier.
__device__ void quantize_block(float *x, int n, int bits, float *red) {
    if (!bits) return;
    float a = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) a = fmaxf(a, fabsf(x[i]));
    a = block_max(a, red);
    if (a == 0.0f) {
        __syncthreads();
        return;
    }
    const int m = (1 << (bits - 1)) - 1;
    const float scale = a / static_cast<float>(m);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float q = rintf(x[i] / scale);
        q = fmaxf(static_cast<float>(-m - 1), fminf(static_cast<float>(m), q));
        x[i] = q * scale;
    }
    __syncthreads();
}

// One butterfly stage of stride H < 64 on a wave's 64 consecutive values:
// the lower element becomes a + b, the upper a - b.
template <int H>
__device__ __forceinline__ float fwht_stage(float x, int lane) {
    const float p = butterfly_partner<H>(x, lane);
    return (lane & H) ? p - x : x + p;
}

// In-place normalised FWHT of v[0..n) in LDS (n a power of two): stages 1..32
// in registers over 64-value chunks, the larger strides through LDS, in the
// reference's stage order. Ends with a barrier.
__device__ void hadamard_block(float *v, int n, float inv) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    int h = 1;
    if (n >= 64) {
        for (int c = wave; c < n / 64; c += waves) {
            float x = v[c * 64 + lane];
            x = fwht_stage<1>(x, lane);
            x = fwht_stage<2>(x, lane);
            x = fwht_stage<4>(x, lane);
            x = fwht_stage<8>(x, lane);
            x = fwht_stage<16>(x, lane);
            x = fwht_stage<32>(x, lane);
            v[c * 64 + lane] = x;
        }
        __syncthreads();
        h = 64;
    }
    for (; h < n; h <<= 1) {
        for (int p = threadIdx.x; p < n / 2; p += blockDim.x) {
            const int j = (p / h) * 2 * h + p % h;
            const float a = v[j], b = v[j + h];
            v[j] = a + b;
            v[j + h] = a - b;
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < n; i += blockDim.x) v[i] *= inv;
    __syncthreads();
}

// The same transform for n = 64 K values with thread i holding value i
// (blockDim = 64 K): stages 1 .. 32 between the lanes of each wave, then
// every thread gathers its column i % 64 + 64 k (k < K) from buf and runs the
// stages 64 .. 32 K on its own copy, keeping entry i / 64: hadamard_block's
// stage order and operands with one barrier (no earlier read of buf may be
// pending). Returns value i.
template <int K>
__device__ __forceinline__ float hadamard_thread(float x, float *buf, float inv) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    x = fwht_stage<1>(x, lane);
    x = fwht_stage<2>(x, lane);
    x = fwht_stage<4>(x, lane);
    x = fwht_stage<8>(x, lane);
    x = fwht_stage<16>(x, lane);
    x = fwht_stage<32>(x, lane);
    buf[threadIdx.x] = x;
    __syncthreads();
    float c[K];
#pragma unroll
    for (int k = 0; k < K; ++k) c[k] = buf[lane + 64 * k];
#pragma unroll
    for (int h = 1; h < K; h <<= 1)
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (!(k & h)) {
                const float a = c[k], b = c[k + h];
                c[k] = a + b;
                c[k + h] = a - b;
            }
    float out = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k)
        if (k == w) out = c[k];
    return out * inv;
}

// engine.cpp:151-180 for an N x N matrix (N <= 8) held by one wave, lane
// l = N i + j holding a[i][j] (lanes past N * N hold copies of lane 0's group
// and never mix into it): row sums over lanes that differ in the low log2(N)
// bits, column sums over the next log2(N) bits (tree sums, not the
// reference's left-to-right ones).
template <int N, int H0, int H1>
__device__ __forceinline__ float lanes_sum(float v, int lane) {
    if constexpr (H0 < H1) {
        v += butterfly_partner<H0>(v, lane);
        return lanes_sum<N, H0 * 2, H1>(v, lane);
    } else {
        return v;
    }
}
template <int H0, int H1>
__device__ __forceinline__ float lanes_max(float v, int lane) {
    if constexpr (H0 < H1) {
        v = fmaxf(v, butterfly_partner<H0>(v, lane));
        return lanes_max<H0 * 2, H1>(v, lane);
    } else {
        return v;
    }
}
template <int H0, int H1>
__device__ __forceinline__ float lanes_min(float v, int lane) {
    if constexpr (H0 < H1) {
        v = fminf(v, butterfly_partner<H0>(v, lane));
        return lanes_min<H0 * 2, H1>(v, lane);
    } else {
        return v;
    }
}

template <int N>
__device__ float sinkhorn_lanes(float a, int lane) {
    constexpr int NN = N * N;
    const float mx = lanes_max<1, NN>(a, lane), mn = lanes_min<1, NN>(a, lane);
    if (!isfinite(mx) || mx - mn > 60.0f) {  // log space (wave-uniform branch)
        for (int it = 0; it < 20; ++it) {
            float m = lanes_max<1, N>(a, lane);
            a -= m + logf(lanes_sum<N, 1, N>(expf(a - m), lane));
            m = lanes_max<N, NN>(a, lane);
            a -= m + logf(lanes_sum<N, N, NN>(expf(a - m), lane));
        }
        return expf(a);
    }
    a = expf(a - mx);
    for (int it = 0; it < 20; ++it) {
        a *= 1.0f / lanes_sum<N, 1, N>(a, lane);
        a *= 1.0f / lanes_sum<N, N, NN>(a, lane);
    }
    return a;
}

// Layer l's residual routing hroute = sinkhorn(hres * a_res[l] + b_res[l])
// (engine.cpp:1034) by wave 0 of a workgroup of its own, which runs beside
// the attention (or gate) workgroups of the launch and takes no part in their
// barriers; the post kernel reads the result.
__device__ void route_wave(const EngineBufs &b, const MhcDev &mh, int l, const EngineDims &d) {
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x, N = d.N, ij = lane % (N * N);
    const float a = b.hres[ij] * mh.a_res[l] + mh.b_res[l * N * N + ij];
    float r;
    switch (N) {
    case 1: r = sinkhorn_lanes<1>(a, lane); break;
    case 2: r = sinkhorn_lanes<2>(a, lane); break;
    case 4: r = sinkhorn_lanes<4>(a, lane); break;
    default: r = sinkhorn_lanes<8>(a, lane); break;
    }
    if (lane < N * N) b.hroute[lane] = r;
}

// Token tok's int8 input of the target's projection from the vector in v
// (position p at v[p - v0]; positions at or past n read as zero): groups
// [g0, g1), one wave per group (prepare_group_wave), waves from w0 on.
__device__ void prepare_groups(PrepTarget pt, const float *v, int v0, int n, int g0, int g1, int w0, int tok,
                               int tokens) {
    const int lane = threadIdx.x & 63, wave = static_cast<int>(threadIdx.x >> 6) - w0;
    const int waves = static_cast<int>(blockDim.x >> 6) - w0;
    if (wave < 0) return;
    int8_t *qv = pt.q + static_cast<size_t>(tok) * pt.dev;
    for (int g = g0 + wave; g < g1; g += waves) {
        const int base = g * pt.group;
        float *xs = pt.xs + static_cast<size_t>(tok) * pt.groups + g;  // stored only for a group before padded
        float *xst = pt.xst ? pt.xst + static_cast<size_t>(g) * tokens + tok : nullptr;
        if (pt.group == 128) {
            float r[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int pos = base + lane + 64 * k;
                r[k] = pos < n ? v[pos - v0] : 0.0f;
            }
            prepare_group_wave<128>(r, lane, base, pt.padded, pt.dev, pt.scale, pt.kind, qv, xs, xst);
        } else {
            float r[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int pos = base + lane + 64 * k;
                r[k] = pos < n ? v[pos - v0] : 0.0f;
            }
            prepare_group_wave<256>(r, lane, base, pt.padded, pt.dev, pt.scale, pt.kind, qv, xs, xst);
        }
    }
}

// x[n][d] = z[d] * sqrt(D) for every lane (engine.cpp:973-974), then nx = rms(x).
__global__ __launch_bounds__(kEngThreads) void eng_start_kernel(const float *__restrict__ z, EngineBufs b0,
                                                                EngineDims d) {
    __shared__ float red[kEngThreads / 64];
    const EngineBufs b = at_token(b0, d, blockIdx.y);
    z += static_cast<size_t>(blockIdx.y) * d.D;
    for (int i = threadIdx.x; i < d.N * d.D; i += blockDim.x) b.x[i] = z[i % d.D] * d.sqrt_d;
    __syncthreads();
    rms_block(b.x, b.nx, d.N * d.D, nullptr, red);
}

// Tables the step does not read become zeros; then the activation quantiser (engine.cpp:760-768).
__global__ __launch_bounds__(kEngThreads) void eng_engram_in_kernel(EngineBufs b0, const StepParams *__restrict__ p,
                                                                    int site, EngineDims d) {
    __shared__ float red[kEngThreads / 64];
    const EngineBufs b = at_token(b0, d, blockIdx.y);
    p += blockIdx.y;
    const int zero = p->engram_zero[site];
    for (int i = threadIdx.x; i < d.D; i += blockDim.x)
        if ((zero >> (i / d.subdim)) & 1) b.e[i] = 0.0f;
    __syncthreads();
    quantize_block(b.e, d.D, d.abits, red);
}

// The dilated causal conv over the taps (engine.cpp:771-780): a tap inside
// this token's chunk reads that token's raw values, an older one the ring.
__global__ __launch_bounds__(kEngThreads) void eng_engram_conv_kernel(EngineBufs b0, const float *__restrict__ taps,
                                                                      const StepParams *__restrict__ p, int site,
                                                                      EngineDims d) {
    const EngineBufs b = at_token(b0, d, blockIdx.y);
    p += blockIdx.y;
    const float *ring = b0.engring + static_cast<size_t>(site) * d.engring * d.D;
    for (int i = threadIdx.x; i < d.D; i += blockDim.x) {
        float sum = 0.0f;
        for (int t = 0; t < d.taps; ++t) {
            const int pos = p->tap_pos[t];
            if (pos < 0) continue;
            const float v = pos >= p->chunk_start
                                ? b0.rawv[static_cast<size_t>(pos - p->chunk_start) * d.D + i]
                                : ring[static_cast<size_t>(pos % d.engring) * d.D + i];
            sum += taps[t * d.D + i] * v;
        }
        b.ev[site * d.D + i] = sum;
    }
}

// Ring rows of the chunk's last min(tokens, engring) positions (block y: one of them).
__global__ __launch_bounds__(kEngThreads) void eng_engram_ring_kernel(EngineBufs b0, const StepParams *__restrict__ p,
                                                                      int site, int tokens, EngineDims d) {
    const int keep = tokens < d.engring ? tokens : d.engring;
    const int t = tokens - keep + static_cast<int>(blockIdx.y);
    float *ring = b0.engring + static_cast<size_t>(site) * d.engring * d.D;
    const int row = p[t].position % d.engring;
    for (int i = threadIdx.x; i < d.D; i += blockDim.x)
        ring[static_cast<size_t>(row) * d.D + i] = b0.rawv[static_cast<size_t>(t) * d.D + i];
}

// Slot of entry s of a token's attention list (engine.cpp:907-909): the
// prefix slots, then positions start.. in the cache ring, which holds `ring`
// positions past the prefix (cache_slot, engine.cpp:500, with a ring of the
// window plus a prompt chunk so a chunk's stores never evict what its earlier
// tokens read).
// SlotMap holds the token's list parameters in registers and computes a slot
// without branches (the ring offset is computed and discarded where unused).
struct SlotMap {
    int prefix_count, start, window, prefix, ring;
    __device__ explicit SlotMap(const StepParams *p)
        : prefix_count(p->prefix_count), start(p->start), window(p->window), prefix(p->prefix),
          ring(p->ring > 0 ? p->ring : 1) {}
    __device__ explicit SlotMap(const StepHead &h)
        : prefix_count(h.prefix_count), start(h.start), window(h.window), prefix(h.prefix),
          ring(h.ring > 0 ? h.ring : 1) {}
    __device__ int operator()(int s) const {
        const int pos = s < prefix_count ? s : start + s - prefix_count;
        const int wrapped = prefix + (pos - prefix) % ring;
        return !window || pos < prefix ? pos : wrapped;
    }
};
__device__ __forceinline__ int slot_at(const StepParams *p, int s) { return SlotMap(p)(s); }

// SlotMap's slots of s0, s0 + step, .. (step > 0) without a division per entry:
// past the prefix entries (pos - prefix) mod ring advances by step mod ring,
// so one remainder is kept and stepped, in straight-line code. Exact for the lists
// GpuEngine::set_token builds, whose prefix entries lie inside the prefix
// (prefix_count <= prefix, so entry s < prefix_count is slot s).
struct SlotWalk {
    SlotMap m;  // a copy (in registers)
    int s, step, rem;  // rem = (start + s - prefix_count - prefix) mod ring, in [0, ring)
    int dstep;         // step mod ring
    __device__ SlotWalk(const SlotMap &map, int s0, int st) : m(map), s(s0), step(st), dstep(st % map.ring) {
        const int u = (m.start + s0 - m.prefix_count - m.prefix) % m.ring;
        rem = u < 0 ? u + m.ring : u;
    }
    __device__ int slot() const {
        const int pos = s < m.prefix_count ? s : m.start + s - m.prefix_count;
        return s < m.prefix_count || !m.window || pos < m.prefix ? pos : m.prefix + rem;
    }
    __device__ void next() {
        s += step;
        rem += dstep;
        rem = rem >= m.ring ? rem - m.ring : rem;
    }
};

struct MixArgs {
    int l, nsites;
    int sites[kEngMaxSites];
    int mhc_row[3];
};

// Lane gates of layer l from its mHC projections proj (LDS: pre [N], post
// [N], res [N * N]) into hp (LDS) and b (engine.cpp:980-986).
// The gate parameters of layer l for lane threadIdx.x < N, loaded ahead of
// mix_gates.
struct GateParams {
    float a_pre, b_pre, a_post, b_post;
};
template <int N>
__device__ __forceinline__ GateParams gate_params(const MhcDev &mh, int l) {
    GateParams g{0.0f, 0.0f, 0.0f, 0.0f};
    if (threadIdx.x < static_cast<unsigned>(N)) {
        const int n = threadIdx.x;
        g = GateParams{mh.a_pre[l], mh.b_pre[l * N + n], mh.a_post[l], mh.b_post[l * N + n]};
    }
    return g;
}
// (lead false: hp only, no store to memory; hpost_out receives the post gates)
template <int N>
__device__ __forceinline__ void mix_gates(const EngineBufs &b, const GateParams &gp, int l, const float *proj,
                                          float *hp, float *hpost_out, bool lead) {
    if (threadIdx.x < static_cast<unsigned>(N)) {
        const int n = threadIdx.x;
        const float pre = proj[n], post = proj[N + n];
        const float hpre = sigmoidf_(gp.a_pre * pre + gp.b_pre + (n == l % N ? 4.0f : -4.0f));
        const float hpost = 2.0f * sigmoidf_(gp.a_post * post + gp.b_post + (n == l % N ? 0.0f : -4.0f));
        hp[n] = hpre;
        if (lead) {
            b.hpre[n] = hpre;
            hpost_out[n] = hpost;
        }
    }
    if (lead)
        for (int i = threadIdx.x; i < N * N; i += blockDim.x) b.hres[i] = proj[2 * N + i];
}

// The engram gates of the layer's sites on bx (engine.cpp:987-991), after a barrier that
// follows the stores of b.u and b.bx. Ends with a barrier.
__device__ void mix_sites(const EngineBufs &b, const MixArgs &m, const EngineDims &d, float *red, float *zs,
                          float *ps) {
    const int D = d.D;
    for (int k = 0; k < m.nsites; ++k) {
        // (a select over the fixed slots: indexing the argument block at run time copies it to scratch)
        int s = m.sites[0];
#pragma unroll
        for (int j = 1; j < kEngMaxSites; ++j)
            if (k == j) s = m.sites[j];
        rms_block(b.u, zs, D, nullptr, red);
        rms_block(b.ek + s * D, ps, D, nullptr, red);
        float dot = 0.0f;
        for (int i = threadIdx.x; i < D; i += blockDim.x) dot += zs[i] * ps[i];
        dot = block_sum(dot, red);
        const float alpha = sigmoidf_(dot / d.sqrt_d);
        for (int i = threadIdx.x; i < D; i += blockDim.x) b.bx[i] += alpha * b.ev[s * D + i];
        __syncthreads();
    }
}

// engine.cpp:980-992: lane gates from the mHC projections, the pre-mixed
// residual u = bx, engram gates, then z = quant(rms(bx) * (1 + norm_in)).
template <int N>
__global__ __launch_bounds__(kEngThreads) void eng_mix_kernel(EngineBufs b0, LayerDev ld, MhcDev mh, MixArgs m,
                                                              EngineDims d, PrepTarget pt) {
    const EngineBufs b = at_token(b0, d, blockIdx.y);
    __shared__ float red[kEngThreads / 64];
    __shared__ float hp[16];
    __shared__ float zs[4096], ps[4096];
    __shared__ float proj[2 * 8 + 64];  // this layer's mHC projections: pre [N], post [N], res [N * N]
    const int D = d.D;
    // (no indexing of b's pointer arrays by a runtime value: that would place b in private memory)
    const float *pre_rows = b.mhc_out[0] + m.mhc_row[0], *post_rows = b.mhc_out[1] + m.mhc_row[1];
    const float *res_rows = b.mhc_out[2] + m.mhc_row[2];
    for (int task = threadIdx.x; task < 2 * N + N * N; task += blockDim.x)
        proj[task] = task < N ? pre_rows[task] : task < 2 * N ? post_rows[task - N] : res_rows[task - 2 * N];
    __syncthreads();
    mix_gates<N>(b, gate_params<N>(mh, m.l), m.l, proj, hp, b.hpost, true);
    __syncthreads();
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        float sum = 0.0f;
#pragma unroll
        for (int n = 0; n < N; ++n) sum += hp[n] * b.x[n * D + i];
        b.u[i] = sum;
        b.bx[i] = sum;
    }
    __syncthreads();
    mix_sites(b, m, d, red, zs, ps);
    rms_block(b.bx, b.z, D, ld.norm_in, red);
    quantize_block(b.z, D, d.abits, red);
    if (pt.q) prepare_groups(pt, b.z, 0, D, 0, pt.dev / pt.group, 0, blockIdx.y, gridDim.y);
}

// engine.cpp:994-1021: per-head rms of q and k, RoPE (first half paired with
// second half), the new token's K/V into its cache slot (fp32, or the int8
// quantiser of kv_store), and the attention slot list.
__global__ __launch_bounds__(kEngThreads) void eng_qk_kernel(EngineBufs b0, LayerDev ld, KvLayer kv,
                                                             const StepParams *__restrict__ p, EngineDims d) {
    struct Args {
        EngineBufs b0;
        LayerDev ld;
        KvLayer kv;
        const StepParams *p;
        EngineDims d;
    };
    touch_kernargs<sizeof(Args)>();
    const EngineBufs b = at_token(b0, d, blockIdx.y);
    p += blockIdx.y;
    const int HD = d.HD, half = HD / 2;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int heads = d.H + d.KV;
    if (HD <= 128 && heads <= static_cast<int>(blockDim.x >> 6)) {
        // one head per wave, every input loaded up front (one pair per lane), and the
        // k-head waves store their rotated K row and the V row into the cache from
        // registers: the same arithmetic as the general form below
        if (wave >= heads) return;
        const int h = wave, kh = h - d.H;
        float *src = h < d.H ? b.q + h * HD : b.k + kh * HD;
        const float *gain = h < d.H ? ld.q_norm : ld.k_norm;
        const float *vr = b.v + (h < d.H ? 0 : kh) * HD;
        const float v0 = load_or_zero(src, HD, lane), v1 = load_or_zero(src, HD, lane + 64);
        const float a0 = load_or_zero(src, half, lane), c0 = load_or_zero(src + half, half, lane);
        const float ga = load_or_zero(gain, half, lane), gc = load_or_zero(gain + half, half, lane);
        const float co = load_or_zero(p->rope_cos, half, lane), si = load_or_zero(p->rope_sin, half, lane);
        const float w0 = load_or_zero(vr, HD, lane), w1 = load_or_zero(vr, HD, lane + 64);
        float ss = 0.0f;
        ss += v0 * v0;
        if (HD > 64) ss += v1 * v1;
        ss = wave_sum(ss, lane);
        const float r = 1.0f / sqrtf(ss / static_cast<float>(HD) + 1e-6f);
        const float a = a0 * r * (1.0f + ga), c = c0 * r * (1.0f + gc);
        const float lo = a * co - c * si, hi = c * co + a * si;  // elements lane and lane + half
        if (lane < half) {
            src[lane] = lo;
            src[lane + half] = hi;
        }
        if (h < d.H) return;
        const size_t row = static_cast<size_t>(kh) * d.capacity + p->slot;
        if (kv.k32) {
            ND_GLOBAL float *kc = (ND_GLOBAL float *)(kv.k32 + row * HD);
            ND_GLOBAL float *vc = (ND_GLOBAL float *)(kv.v32 + row * HD);
            if (lane < half) {
                kc[lane] = lo;
                kc[lane + half] = hi;
            }
            if (lane < HD) vc[lane] = w0;
            if (lane + 64 < HD) vc[lane + 64] = w1;
        } else {
            const float mk = wave_max(lane < half ? fmaxf(fabsf(lo), fabsf(hi)) : 0.0f, lane);
            const float mv = wave_max(fmaxf(fabsf(w0), fabsf(w1)), lane);
            const float sk = mk > 0 ? mk / 127.0f : 1.0f, sv = mv > 0 ? mv / 127.0f : 1.0f;
            const float ik = mk > 0 ? 127.0f / mk : 0.0f, iv = mv > 0 ? 127.0f / mv : 0.0f;
            if (lane == 0) {
                kv.ks[row] = sk;
                kv.vs[row] = sv;
            }
            auto q8 = [](float x, float inv) {
                return static_cast<int8_t>(fmaxf(-127.0f, fminf(127.0f, rintf(x * inv))));
            };
            if (lane < half) {
                kv.k8[row * HD + lane] = q8(lo, ik);
                kv.k8[row * HD + lane + half] = q8(hi, ik);
            }
            if (lane < HD) kv.v8[row * HD + lane] = q8(w0, iv);
            if (lane + 64 < HD) kv.v8[row * HD + lane + 64] = q8(w1, iv);
        }
        return;
    }
    for (int h = wave; h < heads; h += blockDim.x >> 6) {  // one wave per head (q heads, then k heads)
        float *src = h < d.H ? b.q + h * HD : b.k + (h - d.H) * HD;
        const float *gain = h < d.H ? ld.q_norm : ld.k_norm;
        float ss = 0.0f;
        for (int i = lane; i < HD; i += 64) ss += src[i] * src[i];
        ss = wave_sum(ss, lane);
        const float r = 1.0f / sqrtf(ss / static_cast<float>(HD) + 1e-6f);
        // lane j rotates the pair (j, j + HD/2): it reads and writes both, nobody else does
        for (int j = lane; j < half; j += 64) {
            const float co = p->rope_cos[j], si = p->rope_sin[j];
            const float a = src[j] * r * (1.0f + gain[j]), c = src[j + half] * r * (1.0f + gain[j + half]);
            src[j] = a * co - c * si;
            src[j + half] = c * co + a * si;
        }
    }
    __syncthreads();
    // the new token's K / V (one wave per kv head)
    const int slot = p->slot;
    for (int kh = wave; kh < d.KV; kh += blockDim.x >> 6) {
        const float *kr = b.k + kh * HD, *vr = b.v + kh * HD;
        const size_t row = static_cast<size_t>(kh) * d.capacity + slot;
        if (kv.k32) {
            for (int i = lane; i < HD; i += 64) {
                kv.k32[row * HD + i] = kr[i];
                kv.v32[row * HD + i] = vr[i];
            }
        } else {
            float mk = 0.0f, mv = 0.0f;
            for (int i = lane; i < HD; i += 64) {
                mk = fmaxf(mk, fabsf(kr[i]));
                mv = fmaxf(mv, fabsf(vr[i]));
            }
            mk = wave_max(mk, lane);
            mv = wave_max(mv, lane);
            const float sk = mk > 0 ? mk / 127.0f : 1.0f, sv = mv > 0 ? mv / 127.0f : 1.0f;
            const float ik = mk > 0 ? 127.0f / mk : 0.0f, iv = mv > 0 ? 127.0f / mv : 0.0f;
            if (lane == 0) {
                kv.ks[row] = sk;
                kv.vs[row] = sv;
            }
            for (int i = lane; i < HD; i += 64) {
                const float qk = fmaxf(-127.0f, fminf(127.0f, rintf(kr[i] * ik)));
                const float qv = fmaxf(-127.0f, fminf(127.0f, rintf(vr[i] * iv)));
                kv.k8[row * HD + i] = static_cast<int8_t>(qk);
                kv.v8[row * HD + i] = static_cast<int8_t>(qv);
            }
        }
    }
}

// The attention step of one kv head in one workgroup: the norms and RoPE of
// its G query heads and of its K head, the new K / V row into the cache (fp32,
// or the int8 store quantiser), attention over the slot list (computed in
// place from the position, engine.cpp:900-909) and the output gate att *=
// sigmoid(gate) (engine.cpp:994-1023). Nothing crosses kv heads, so one
// launch does it all.

// The scores [G][length] live in LDS, or, past the LDS budget (long
// contexts), in `scores` ([tokens][kv heads][G][max_length] in device memory):
// the same block writes, reduces and reads them, ordered by its barriers.
// I8: an int8 KV cache (codes with a scale per row, the store kernel's
// quantiser for the new row): s = dot(q, float(k8)) * k_scale * (1 /
// sqrt(head_dim)), p = softmax(s), out = sum_s (p_s * v_scale_s) * float(v8)
// (engine.cpp:898-967, as the int8 attention kernel).
// WIDE (without PREPARED): head_dim above 128 or more heads than waves (G + 1
// > 4); otherwise each wave normalises one head from registers loaded ahead
// of the K prefetch.
template <bool PREPARED, bool GLOBAL_SCORES, bool I8, bool WIDE = false>
__global__ __launch_bounds__(256) void eng_attn_fused_kernel(EngineBufs b0, LayerDev ld, KvLayer kv,
                                                             const StepParams *__restrict__ p, StepHead sh,
                                                             EngineDims d, float *__restrict__ scores, int max_length,
                                                             MhcDev mh, int layer, PrepTarget pt, OutProj op) {
    struct Args {
        EngineBufs b0;
        LayerDev ld;
        KvLayer kv;
        const StepParams *p;
        StepHead sh;
        EngineDims d;
        float *scores;
        int max_length;
        MhcDev mh;
        int layer;
        PrepTarget pt;
    };
    touch_kernargs<offsetof(Args, pt)>();
    const int split = op.codes ? op.split_shift : 0;  // workgroups per kv head: 1 << split
    if (blockIdx.x == (d.KV << split)) {  // the routing workgroup
        route_wave(at_token(b0, d, blockIdx.y), mh, layer, d);
        return;
    }
    constexpr int kMaxG = 8, kPre = 8, kWaves = 4;
    extern __shared__ float sc_lds[];  // [G][length] when the scores fit
    __shared__ float qs[8 * 1024];  // query heads, then the partial outputs [R][G][HD] (1024 G floats)
    __shared__ float red[kMaxG * kWaves], red2[kMaxG * kWaves];
    __shared__ float knew_scale, vnew_scale;  // int8: the new K / V rows' scales
    const EngineBufs b = at_token(b0, d, blockIdx.y);
    p += blockIdx.y;
    const int kh = blockIdx.x >> split, part = blockIdx.x & ((1 << split) - 1);
    const int G = d.H / d.KV, HD = d.HD, half = HD / 2, t = threadIdx.x;
    float *sc = GLOBAL_SCORES
                    ? scores + (static_cast<size_t>(blockIdx.y) * d.KV + kh) * G * static_cast<size_t>(max_length)
                    : sc_lds;
    // one token (not PREPARED): the slot list from the kernel arguments
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63, length = PREPARED ? p->length : sh.length;
    const int my_slot = PREPARED ? p->slot : sh.slot;  // this token's cache slot
    const size_t row0 = static_cast<size_t>(kh) * d.capacity;  // this kv head's first cache row
    const float *kc = I8 ? nullptr : kv.k32 + row0 * HD;
    const float *vc = I8 ? nullptr : kv.v32 + row0 * HD;
    const int8_t *kc8 = I8 ? kv.k8 + row0 * HD : nullptr;
    const int8_t *vc8 = I8 ? kv.v8 + row0 * HD : nullptr;
    const float *ksc = I8 ? kv.ks + row0 : nullptr;
    const float *vsc = I8 ? kv.vs + row0 : nullptr;
    // loaded before the norms: the output gate of output t, and at head_dim 64 the K row of this thread's
    // first slot unless this kernel stores that row below (the new token's)
    // (loads without branches: an entry past the list reads slot 0 and is not used)
    const SlotMap slot_of = PREPARED ? SlotMap(p) : SlotMap(sh);
    const float gate_t = load_or_zero(b.gate + kh * G * HD, G * HD, t);
    // The inputs of this wave's first norm / RoPE head (h = wave <= G, head_dim
    // <= 128: one RoPE pair per lane) and the new V row, loaded before the K
    // prefetch below so that waiting for them does not wait for it.
    float nv0 = 0.0f, nv1 = 0.0f, na = 0.0f, nc = 0.0f, nga = 0.0f, ngc = 0.0f, nco = 0.0f, nsi = 0.0f;
    float vnew = 0.0f;
    // PREPARED: this thread's query value (G * HD <= 256: one per thread), loaded ahead of the prefetch too
    const float qpre = PREPARED ? load_or_zero(b.q + kh * G * HD, G * HD, t) : 0.0f;
    if constexpr (!PREPARED && !WIDE) {  // (every wave loads, without a branch, so the waits below stay exact)
        const int h = wave <= G ? wave : G;
        const float *src = h < G ? b.q + (kh * G + h) * HD : b.k + kh * HD;
        const float *gain = h < G ? ld.q_norm : ld.k_norm;
        nv0 = load_or_zero(src, HD, lane);
        nv1 = load_or_zero(src, HD, lane + 64);
        na = load_or_zero(src, half, lane);
        nc = load_or_zero(src + half, half, lane);
        nga = load_or_zero(gain, half, lane);
        ngc = load_or_zero(gain + half, half, lane);
        nco = load_or_zero(p->rope_cos, half, lane);
        nsi = load_or_zero(p->rope_sin, half, lane);
        if (!I8) vnew = load_or_zero(b.v + kh * HD, HD, t);
    }
    const int slot_t = t < length ? slot_of(t) : 0;
    const bool k_early = HD == 64 && t < length && (PREPARED || slot_t != my_slot);
    float4 kpre[I8 ? 4 : 16];  // fp32: the row; int8: its 64 codes
    float kpre_s = 0.0f;
    {  // buffer loads over this kv head's rows (nothing unless head_dim is 64; a thread past the list
       // reads zeros without a memory request), without a branch
        // (uniform: readfirstlane keeps the buffer descriptor in scalar registers)
        const uint32_t rows = __builtin_amdgcn_readfirstlane(HD == 64 ? static_cast<uint32_t>(d.capacity) : 0u);
        const uint32_t row = t < length ? static_cast<uint32_t>(slot_t) : 0x00800000u;  // past any cache
        if constexpr (I8) {
            const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(kc8, rows * 64u);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                kpre[c] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, row * 64u, c * 16, 0));
            kpre_s = load_or_zero(ksc, static_cast<int>(rows), static_cast<int>(row));
        } else {
            const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(kc, rows * 256u);
#pragma unroll
            for (int c = 0; c < 16; ++c)
                kpre[c] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, row * 256u, c * 16, 0));
        }
    }
    // values: thread t takes 16-byte column c = t % (HD / 4) of the V rows of slots r, r + R, ..
    // (r = t / (HD / 4), R = 256 / (HD / 4) subsets), so its loads are all in flight together; the R
    // partial sums per output then add up in subset order. When HD / 4 does not divide 256 the last
    // threads (r == R) take no slots and write no partials: R * G * HD <= 1024 G floats fit in qs.
    const int cols4 = HD / 4, R = blockDim.x / cols4, c4 = t % cols4, r = t / cols4;
    const bool sub = r < R;
    const uint32_t esz = I8 ? 1u : 4u;
    // The one-slot form below (head_dim 64) takes every V row of the thread (2 kPre) and its int8
    // scale here, ahead of the norms: the new token's row (not stored yet) is marked in vnew_rows and
    // read from LDS instead. Other head sizes read nothing (an empty resource).
    constexpr bool kOneSlotForm = !GLOBAL_SCORES && (PREPARED || !WIDE);
    float4 vall[kOneSlotForm && !I8 ? 2 * kPre : 1];
    uint32_t vall8[kOneSlotForm && I8 ? 2 * kPre : 1];  // int8: the four codes (converted where used)
    float vsr[kOneSlotForm && I8 ? 2 * kPre : 1];
    uint32_t vnew_rows = 0;
    if constexpr (kOneSlotForm) {
        // (uniform: readfirstlane keeps the buffer descriptor in scalar registers)
        const uint32_t rows = __builtin_amdgcn_readfirstlane(HD == 64 ? static_cast<uint32_t>(d.capacity) : 0u);
        const __amdgpu_buffer_rsrc_t ve =
            buffer_rsrc(I8 ? static_cast<const void *>(vc8) : static_cast<const void *>(vc), rows * 64u * esz);
        const int new_slot = PREPARED ? -1 : my_slot;
        SlotWalk wk(slot_of, r, R);
#pragma unroll
        for (int k = 0; k < 2 * kPre; ++k, wk.next()) {
            const int s = r + k * R;
            const int sl = wk.slot();
            const bool live = sub && s < length;
            vnew_rows |= live && sl == new_slot ? 1u << k : 0u;
            const uint32_t off = live ? (static_cast<uint32_t>(sl) * 64u + 4u * c4) * esz : 0xFFFFFFF0u;
            if constexpr (I8) {
                vall8[k] = __builtin_amdgcn_raw_buffer_load_b32(ve, off, 0, 0);
                vsr[k] = load_or_zero(vsc, static_cast<int>(rows), live ? sl : static_cast<int>(rows));
            } else {
                vall[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ve, off, 0, 0));
            }
        }
    }
    // eng_qk_kernel's quantiser for the new K / V rows (same codes and scales), by
    // the wave that wrote the rotated K row to kw (LDS); with kq, the K codes (as
    // floats) and their scale also go to LDS (kq, knew_scale) for the scores
    auto quantize_new_kv = [&](const float *kw, float *kq) {
        const float *vr = b.v + kh * HD;
        const size_t row = row0 + my_slot;
        float mk = 0.0f, mv = 0.0f;
        for (int i = lane; i < HD; i += 64) {
            mk = fmaxf(mk, fabsf(kw[i]));
            mv = fmaxf(mv, fabsf(vr[i]));
        }
        mk = wave_max(mk, lane);
        mv = wave_max(mv, lane);
        const float sk = mk > 0 ? mk / 127.0f : 1.0f, sv = mv > 0 ? mv / 127.0f : 1.0f;
        const float ik = mk > 0 ? 127.0f / mk : 0.0f, iv = mv > 0 ? 127.0f / mv : 0.0f;
        if (lane == 0) {
            kv.ks[row] = sk;
            kv.vs[row] = sv;
            if (kq) {
                knew_scale = sk;
                vnew_scale = sv;
            }
        }
        for (int i = lane; i < HD; i += 64) {
            const float qk = fmaxf(-127.0f, fminf(127.0f, rintf(kw[i] * ik)));
            const float qv = fmaxf(-127.0f, fminf(127.0f, rintf(vr[i] * iv)));
            kv.k8[row * HD + i] = static_cast<int8_t>(qk);
            kv.v8[row * HD + i] = static_cast<int8_t>(qv);
            if (kq) {
                kq[i] = qk;
                kq[HD + i] = qv;  // the V codes, after the K codes
            }
        }
    };
    if (PREPARED) {  // eng_qk normalised and rotated q and stored K / V
        if (G * HD <= static_cast<int>(blockDim.x)) {
            if (t < G * HD) qs[t] = qpre;
        } else {
            for (int i = t; i < G * HD; i += blockDim.x) qs[i] = b.q[kh * G * HD + i];
        }
    } else if constexpr (!WIDE) {
        // norms + RoPE, one head per wave on the preloaded values (straight-line
        // code, LDS and global stores apart, so nothing here waits for the
        // prefetch above): heads 0..G-1 are this block's query heads (into qs),
        // head G its K row (into the cache; int8: into LDS, then through the
        // store kernel's quantiser)
        if (wave <= G) {
            float ss = 0.0f;
            ss += nv0 * nv0;
            if (HD > 64) ss += nv1 * nv1;
            ss = wave_sum(ss, lane);
            const float r = 1.0f / sqrtf(ss / static_cast<float>(HD) + 1e-6f);
            const float a = na * r * (1.0f + nga), c = nc * r * (1.0f + ngc);
            const float lo = a * nco - c * nsi, hi = c * nco + a * nsi;
            if (wave < G) {
                if (lane < half) {
                    qs[wave * HD + lane] = lo;
                    qs[wave * HD + lane + half] = hi;
                }
            } else if constexpr (I8) {
                float *kw = qs + kMaxG * HD;
                if (lane < half) {
                    kw[lane] = lo;
                    kw[lane + half] = hi;
                }
                __builtin_amdgcn_wave_barrier();
                quantize_new_kv(kw, qs + (kMaxG + 1) * HD);
            } else {
                ND_GLOBAL float *kw = (ND_GLOBAL float *)(kv.k32 + (row0 + my_slot) * HD);
                float *knew = qs + kMaxG * HD;  // the new row for the scores, from LDS
                if (lane < half) {
                    kw[lane] = lo;
                    kw[lane + half] = hi;
                    knew[lane] = lo;
                    knew[lane + half] = hi;
                }
            }
        }
        if (!I8 && t < HD) {
            ((ND_GLOBAL float *)kv.v32)[(row0 + my_slot) * HD + t] = vnew;
            qs[(kMaxG + 2) * HD + t] = vnew;  // the new V row for the values, from LDS
        }
    } else {
    // the general form: any head_dim, several heads per wave
    float *kw = I8 ? qs + kMaxG * HD : kv.k32 + row0 * HD + static_cast<size_t>(my_slot) * HD;
    for (int h = wave; h <= G; h += blockDim.x >> 6) {
        const float *src = h < G ? b.q + (kh * G + h) * HD : b.k + kh * HD;
        const float *gain = h < G ? ld.q_norm : ld.k_norm;
        float *dst = h < G ? qs + h * HD : kw;
        float ss = 0.0f;
        for (int i = lane; i < HD; i += 64) ss += src[i] * src[i];
        ss = wave_sum(ss, lane);
        const float r = 1.0f / sqrtf(ss / static_cast<float>(HD) + 1e-6f);
        for (int j = lane; j < half; j += 64) {
            const float co = p->rope_cos[j], si = p->rope_sin[j];
            const float a = src[j] * r * (1.0f + gain[j]), c = src[j + half] * r * (1.0f + gain[j + half]);
            dst[j] = a * co - c * si;
            dst[j + half] = c * co + a * si;
        }
        if (I8 && h == G) quantize_new_kv(kw, nullptr);
    }
    if (!I8)
        for (int i = t; i < HD; i += blockDim.x) kv.v32[(row0 + my_slot) * HD + i] = b.v[kh * HD + i];
    }
    __syncthreads();
    // V loads are buffer loads: an entry past the list reads zeros (offset past the resource)
    const __amdgpu_buffer_rsrc_t vres = buffer_rsrc(I8 ? static_cast<const void *>(vc8) : static_cast<const void *>(vc),
                                                    static_cast<uint32_t>(d.capacity) * HD * esz);
    auto load_v = [&](int s) -> float4 {
        const uint32_t off =
            sub && s < length ? (static_cast<uint32_t>(slot_of(s)) * HD + 4u * c4) * esz : 0xFFFFFFF0u;
        if constexpr (I8) return int8x4_to_float4(__builtin_amdgcn_raw_buffer_load_b32(vres, off, 0, 0));
        else return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(vres, off, 0, 0));
    };
    float4 acc[kMaxG];
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) acc[g] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // One slot per thread (head_dim 64, scores in LDS, the new K row in LDS or
    // none): the scores stay in registers through the block max and sum (two
    // barriers), the probabilities p = e * (1 / sum) are formed where the values
    // use them, and every V row of the thread (2 kPre for head_dim 64) is loaded
    // before the softmax. Same arithmetic and order as the general form below.
    const bool one_slot = kOneSlotForm && HD == 64 && length <= static_cast<int>(blockDim.x);
    // GG: heads per kv head when it is 1, 2 or 4 (straight-line code over the
    // heads); kMaxG: G at run time (heads past G skipped)
    auto one_slot_form = [&](auto gc) {
        constexpr int GG = decltype(gc)::value;
        auto head = [&](int g) { return GG < kMaxG || g < G; };
        float sv[GG];  // scores of slot t (-inf past the list, as the max's start value)
#pragma unroll
        for (int g = 0; g < GG; ++g) sv[g] = -INFINITY;
        if (t < length) {
            // the prefetched row, or for the new token's slot (not prefetched) the row written to LDS above
            float4 kf[16];
            float kscale = 1.0f;
            if (k_early) {
                if constexpr (I8) {
#pragma unroll
                    for (int c = 0; c < 16; ++c) kf[c] = int8x4_to_float4(__builtin_bit_cast(u32x4, kpre[c / 4])[c % 4]);
                    kscale = kpre_s;
                } else {
#pragma unroll
                    for (int c = 0; c < 16; ++c) kf[c] = kpre[c];
                }
            } else {
                const float4 *kn = reinterpret_cast<const float4 *>(qs + (I8 ? kMaxG + 1 : kMaxG) * HD);
#pragma unroll
                for (int c = 0; c < 16; ++c) kf[c] = kn[c];
                if constexpr (I8) kscale = knew_scale;
            }
#pragma unroll
            for (int g = 0; g < GG; ++g)
                if (head(g)) {
                    const float *q = qs + g * HD;
                    float dot = 0.0f;
#pragma unroll
                    for (int c = 0; c < 16; ++c) {
                        dot += q[4 * c] * kf[c].x;
                        dot += q[4 * c + 1] * kf[c].y;
                        dot += q[4 * c + 2] * kf[c].z;
                        dot += q[4 * c + 3] * kf[c].w;
                    }
                    sv[g] = fmaxf(-INFINITY, I8 ? dot * kscale * d.scale : dot * d.scale);
                }
        }
#pragma unroll
        for (int g = 0; g < GG; ++g)
            if (head(g)) {
                const float mx = wave_max(sv[g], lane);
                if (lane == 0) red[g * kWaves + wave] = mx;
            }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < GG; ++g)
            if (head(g)) {
                float m = red[g * kWaves];
                for (int w = 1; w < kWaves; ++w) m = fmaxf(m, red[g * kWaves + w]);
                const float e = t < length ? expf(sv[g] - m) : 0.0f;
                if (t < length) sc[g * length + t] = e;
                const float den = wave_sum(e, lane);
                if (lane == 0) red2[g * kWaves + wave] = den;
            }
        __syncthreads();
        float inv[GG];
#pragma unroll
        for (int g = 0; g < GG; ++g) {
            inv[g] = 0.0f;
            if (head(g)) {
                float sum = 0.0f;
                for (int w = 0; w < kWaves; ++w) sum += red2[g * kWaves + w];
                inv[g] = 1.0f / sum;
            }
        }
        // the new token's V row (and int8 scale) as this block wrote it, from LDS
        const float4 vnew4 = reinterpret_cast<const float4 *>(qs + (kMaxG + 2) * HD)[c4];
        const float vnew_s = I8 ? vnew_scale : 0.0f;
        auto row = [&](int k) {  // k: a compile-time row index after unrolling
            const int s = r + k * R;
            const bool use = sub && s < length;
            const bool nw = (vnew_rows >> k) & 1u;
            float4 v;
            if constexpr (I8) v = nw ? vnew4 : int8x4_to_float4(vall8[k]);
            else v = nw ? vnew4 : vall[k];
#pragma unroll
            for (int g = 0; g < GG; ++g)
                if (head(g)) {
                    // (read without a branch, so the reads of all rows are in flight together)
                    float pr = sc[g * length + (use ? s : 0)] * inv[g];
                    if constexpr (I8) pr = pr * (nw ? vnew_s : vsr[k]);  // p_s * v_scale_s
                    pr = use ? pr : 0.0f;
                    acc[g].x += pr * v.x;
                    acc[g].y += pr * v.y;
                    acc[g].z += pr * v.z;
                    acc[g].w += pr * v.w;
                }
        };
#pragma unroll
        for (int k = 0; k < kPre; ++k) row(k);
        if (sub && r + kPre * R < length) {
#pragma unroll
            for (int k = kPre; k < 2 * kPre; ++k) row(k);
        }
    };
    if (one_slot) {
        if (G == 1) one_slot_form(std::integral_constant<int, 1>{});
        else if (G == 2) one_slot_form(std::integral_constant<int, 2>{});
        else if (G == 4) one_slot_form(std::integral_constant<int, 4>{});
        else one_slot_form(std::integral_constant<int, kMaxG>{});
    } else {
    float4 vpre[kPre];
#pragma unroll
    for (int k = 0; k < kPre; ++k) vpre[k] = load_v(r + k * R);
    if constexpr (I8) {
        for (int s = t; s < length; s += blockDim.x) {
            const int sl = slot_of(s);
            if (HD == 64) {
                u32x4 k4[4];
                float kscale;
                if (s == t && k_early) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) k4[c] = __builtin_bit_cast(u32x4, kpre[c]);
                    kscale = kpre_s;
                } else {
                    const u32x4 *src = reinterpret_cast<const u32x4 *>(kc8 + static_cast<size_t>(sl) * HD);
#pragma unroll
                    for (int c = 0; c < 4; ++c) k4[c] = src[c];
                    kscale = ksc[sl];
                }
                for (int g = 0; g < G; ++g) {
                    const float *q = qs + g * HD;
                    float dot = 0.0f;
#pragma unroll
                    for (int c = 0; c < 16; ++c) {
                        const float4 k = int8x4_to_float4(k4[c / 4][c % 4]);
                        dot += q[4 * c] * k.x;
                        dot += q[4 * c + 1] * k.y;
                        dot += q[4 * c + 2] * k.z;
                        dot += q[4 * c + 3] * k.w;
                    }
                    sc[g * length + s] = dot * kscale * d.scale;
                }
            } else {
                const uint32_t *k4 = reinterpret_cast<const uint32_t *>(kc8 + static_cast<size_t>(sl) * HD);
                const float kscale = ksc[sl];
                for (int g = 0; g < G; ++g) {
                    const float *q = qs + g * HD;
                    float dot = 0.0f;
                    for (int c = 0; c < HD / 4; ++c) {
                        const float4 k = int8x4_to_float4(k4[c]);
                        dot += q[4 * c] * k.x;
                        dot += q[4 * c + 1] * k.y;
                        dot += q[4 * c + 2] * k.z;
                        dot += q[4 * c + 3] * k.w;
                    }
                    sc[g * length + s] = dot * kscale * d.scale;
                }
            }
        }
    } else if (HD == 64) {
        for (int s = t; s < length; s += blockDim.x) {
            float4 k[16];
            if (s == t && k_early) {
#pragma unroll
                for (int c = 0; c < 16; ++c) k[c] = kpre[c];
            } else {
                const float4 *k4 = reinterpret_cast<const float4 *>(kc + static_cast<size_t>(slot_of(s)) * HD);
#pragma unroll
                for (int c = 0; c < 16; ++c) k[c] = k4[c];
            }
            for (int g = 0; g < G; ++g) {
                const float *q = qs + g * HD;
                float dot = 0.0f;
#pragma unroll
                for (int c = 0; c < 16; ++c) {
                    dot += q[4 * c] * k[c].x;
                    dot += q[4 * c + 1] * k[c].y;
                    dot += q[4 * c + 2] * k[c].z;
                    dot += q[4 * c + 3] * k[c].w;
                }
                sc[g * length + s] = dot * d.scale;
            }
        }
    } else {
        for (int s = t; s < length; s += blockDim.x) {
            const float4 *k4 = reinterpret_cast<const float4 *>(kc + static_cast<size_t>(slot_of(s)) * HD);
            for (int g = 0; g < G; ++g) {
                const float *q = qs + g * HD;
                float dot = 0.0f;
                for (int c = 0; c < HD / 4; ++c) {
                    const float4 k = k4[c];
                    dot += q[4 * c] * k.x;
                    dot += q[4 * c + 1] * k.y;
                    dot += q[4 * c + 2] * k.z;
                    dot += q[4 * c + 3] * k.w;
                }
                sc[g * length + s] = dot * d.scale;
            }
        }
    }
    __syncthreads();
    // softmax of the G heads' rows together: block_max, then block_sum, in their
    // orders (per thread over its slots, the wave's butterfly, the waves in order)
    float mx[kMaxG], den[kMaxG];
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) {
        mx[g] = -INFINITY;
        if (g < G) {
            for (int s = t; s < length; s += blockDim.x) mx[g] = fmaxf(mx[g], sc[g * length + s]);
            mx[g] = wave_max(mx[g], lane);
        }
    }
    if (lane == 0)
#pragma unroll
        for (int g = 0; g < kMaxG; ++g)
            if (g < G) red[g * kWaves + wave] = mx[g];
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) {
        den[g] = 0.0f;
        if (g < G) {
            float m = red[g * kWaves];
            for (int w = 1; w < kWaves; ++w) m = fmaxf(m, red[g * kWaves + w]);
            for (int s = t; s < length; s += blockDim.x) {
                const float e = expf(sc[g * length + s] - m);
                sc[g * length + s] = e;
                den[g] += e;
            }
            den[g] = wave_sum(den[g], lane);
        }
    }
    __syncthreads();
    if (lane == 0)
#pragma unroll
        for (int g = 0; g < kMaxG; ++g)
            if (g < G) red[g * kWaves + wave] = den[g];
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kMaxG; ++g)
        if (g < G) {
            float sum = 0.0f;
            for (int w = 0; w < kWaves; ++w) sum += red[g * kWaves + w];
            const float inv = 1.0f / sum;
            for (int s = t; s < length; s += blockDim.x) {
                const float pr = sc[g * length + s] * inv;
                sc[g * length + s] = I8 ? pr * vsc[slot_of(s)] : pr;  // int8: p_s * v_scale_s
            }
        }
    __syncthreads();
    // rows s0, s0 + R, .. in slot order from registers: an entry past the list adds 0 * 0 (its
    // probability and its zero row)
    auto accumulate_rows = [&](int s0, const float4 (&v)[kPre]) {
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            const int s = s0 + k * R;
            const bool use = sub && s < length;
#pragma unroll
            for (int g = 0; g < kMaxG; ++g)
                if (g < G) {
                    const float pr = use ? sc[g * length + s] : 0.0f;
                    acc[g].x += pr * v[k].x;
                    acc[g].y += pr * v[k].y;
                    acc[g].z += pr * v[k].z;
                    acc[g].w += pr * v[k].w;
                }
        }
    };
    accumulate_rows(r, vpre);
    // the rest kPre rows at a time, every load of a batch in flight together
    for (int s0 = r + kPre * R; sub && s0 < length; s0 += kPre * R) {
#pragma unroll
        for (int k = 0; k < kPre; ++k) vpre[k] = load_v(s0 + k * R);
        accumulate_rows(s0, vpre);
    }
    }
    // OutProj: this thread's rows part * rp + t and + 256 of the out-projection (rp rows per part), the 128
    // positions of this kv head's group (4 code chunks of 4-bit codes, or 2 of 2-bit, plus the next group's 2
    // unused), and their norms, requested ahead of the output phase (rows past the part or the matrix, or no
    // OutProj: an empty resource, zeros)
    constexpr int kOpRows = 2;
    u32x4 opc[kOpRows][4];
    uint32_t opn[kOpRows];
    const int rp = (op.rows + (1 << split) - 1) >> split;
    {
        const int cpg = op.kind == 0 ? 4 : 2;  // code chunks per group of 128 positions
        const uint32_t tiles = op.codes ? static_cast<uint32_t>((op.rows + 255) / 256) : 0u;
        const __amdgpu_buffer_rsrc_t rc = buffer_rsrc(op.codes, __builtin_amdgcn_readfirstlane(tiles * op.chunks * 4096u));
        const __amdgpu_buffer_rsrc_t rn = buffer_rsrc(op.norms, __builtin_amdgcn_readfirstlane(tiles * op.groups * 512u));
#pragma unroll
        for (int j = 0; j < kOpRows; ++j) {
            const int row = part * rp + t + 256 * j;
            const uint32_t tile = static_cast<uint32_t>(row >> 8), rr = static_cast<uint32_t>(row & 255);
            const uint32_t live = t + 256 * j < rp && row < op.rows ? 0u : 0x40000000u;  // else past the resource
#pragma unroll
            for (int c = 0; c < 4; ++c)
                opc[j][c] = __builtin_amdgcn_raw_buffer_load_b128(
                    rc, live | (((tile * op.chunks + static_cast<uint32_t>(kh * cpg + c)) * 256u + rr) * 16u), 0, 0);
            opn[j] = __builtin_amdgcn_raw_buffer_load_b16(
                rn, live | (((tile * op.groups + static_cast<uint32_t>(kh)) * 256u + rr) * 2u), 0, 0);
        }
    }
    float4 *wpart = reinterpret_cast<float4 *>(qs);  // [R][G][HD / 4]: R * G * HD = 1024 G floats
    __syncthreads();
#pragma unroll
    for (int g = 0; g < kMaxG; ++g)
        if (sub && g < G) wpart[(r * G + g) * cols4 + c4] = acc[g];
    __syncthreads();
    float out_t = 0.0f;  // output t (with a target, G * HD <= 256: one output per thread)
    for (int o = t; o < G * HD; o += blockDim.x) {
        const float *wp = reinterpret_cast<const float *>(wpart);
        float a = 0.0f;
        for (int k = 0; k < R; ++k) a += wp[k * G * HD + o];
        const float val = a * sigmoidf_(o == t ? gate_t : b.gate[kh * G * HD + o]);
        if (part == 0) b.att[kh * G * HD + o] = val;
        if (o == t) out_t = val;
    }
    if (pt.q) {  // this kv head's outputs are one group of the out-projection's int8 input
        float *stage = qs;
        __syncthreads();  // every partial read
        if (t < G * HD) stage[t] = out_t;
        __syncthreads();
        prepare_groups(pt, stage, kh * G * HD, d.H * HD, kh, kh + 1, 0, blockIdx.y, gridDim.y);
    }
    if (op.codes) {  // OutProj (G * HD == 128): this kv head's group terms of every out-projection row
        float *stage = qs, *T = qs + 256;
        __syncthreads();  // every partial read
        // the GEMV's in-kernel FWHT of the group (thread t: position t; stages 1 .. 32 in the wave, 64
        // through LDS; the same butterflies and operands), then * 1 / sqrt(128)
        float x = t < 128 ? out_t : 0.0f;
        wave_butterflies<128, 1>(x, lane);
        stage[t] = x;
        __syncthreads();
        const float o = stage[t ^ 64];
        x = o + ((t & 64) ? -x : x);
        x = x * op.scale;
        // the product table (the GEMV kernels' layout): 4-bit, slot p = position p, entry c = cb[c] * rot_p at
        // a 17-float stride; 2-bit, slot s = positions 2s, 2s + 1, entry c0 | c1 << 2 = (cb[c0] * rot_2s,
        // cb[c1] * rot_2s+1) at a 36-float stride
        if (op.kind == 0) {
            if (t < 128)
#pragma unroll
                for (int c = 0; c < 16; ++c) T[t * 17 + c] = op.lut[c] * x;
        } else {
            const int l = lane & 31;
            const float r0 = __shfl(x, 2 * l), r1 = __shfl(x, 2 * l + 1);
            if (t < 128 && lane < 32) {
                float p0[4], p1[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    p0[c] = op.lut[c] * r0;
                    p1[c] = op.lut[c] * r1;
                }
                float4 *dst = reinterpret_cast<float4 *>(T + ((t & ~63) / 2 + l) * 36);
#pragma unroll
                for (int hi = 0; hi < 4; ++hi) {
                    dst[2 * hi] = make_float4(p0[0], p1[hi], p0[1], p1[hi]);
                    dst[2 * hi + 1] = make_float4(p0[2], p1[hi], p0[3], p1[hi]);
                }
            }
        }
        __syncthreads();
        // each row's group sum over the 128 positions in order, times its half norm
        float *parts = op.parts + (static_cast<size_t>(blockIdx.y) * d.KV + kh) * op.rows;
#pragma unroll
        for (int j = 0; j < kOpRows; ++j) {
            const int row = part * rp + t + 256 * j;
            if (256 * j + (t & ~63) >= rp) continue;  // (wave-uniform) no row of this part here
            float gd = 0.0f;
            if (op.kind == 0) {
#pragma unroll
                for (int dw = 0; dw < 16; ++dw) {
                    const uint32_t w = opc[j][dw >> 2][dw & 3];
#pragma unroll
                    for (int i = 0; i < 8; ++i) gd += T[(8 * dw + i) * 17 + ((w >> (4 * i)) & 15u)];
                }
            } else {
#pragma unroll
                for (int dw = 0; dw < 8; ++dw) {
                    const uint32_t w = opc[j][dw >> 2][dw & 3];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const float2 e = *reinterpret_cast<const float2 *>(T + (8 * dw + i) * 36 + 2 * ((w >> (4 * i)) & 15u));
                        gd += e.x;
                        gd += e.y;
                    }
                }
            }
            if (t + 256 * j < rp && row < op.rows) parts[row] = gd * h2f(static_cast<uint16_t>(opn[j]));
        }
    }
}

// Imported K / V rows [count][kvheads][head_dim] into cache slots[count] of
// one layer, fp32 or through the step's int8 quantiser (engine.cpp:788-811):
// one wave per (row, kv head).
__global__ __launch_bounds__(64) void eng_kv_import_kernel(const float *__restrict__ k, const float *__restrict__ v,
                                                           const int *__restrict__ slots, KvLayer kv, EngineDims d) {
    const int t = blockIdx.x / d.KV, kh = blockIdx.x % d.KV, lane = threadIdx.x, HD = d.HD;
    const float *kr = k + (static_cast<size_t>(t) * d.KV + kh) * HD, *vr = v + (static_cast<size_t>(t) * d.KV + kh) * HD;
    const size_t row = static_cast<size_t>(kh) * d.capacity + slots[t];
    if (kv.k32) {
        for (int i = lane; i < HD; i += 64) {
            kv.k32[row * HD + i] = kr[i];
            kv.v32[row * HD + i] = vr[i];
        }
        return;
    }
    float mk = 0.0f, mv = 0.0f;
    for (int i = lane; i < HD; i += 64) {
        mk = fmaxf(mk, fabsf(kr[i]));
        mv = fmaxf(mv, fabsf(vr[i]));
    }
    mk = wave_max(mk, lane);
    mv = wave_max(mv, lane);
    const float ik = mk > 0 ? 127.0f / mk : 0.0f, iv = mv > 0 ? 127.0f / mv : 0.0f;
    if (lane == 0) {
        kv.ks[row] = mk > 0 ? mk / 127.0f : 1.0f;
        kv.vs[row] = mv > 0 ? mv / 127.0f : 1.0f;
    }
    for (int i = lane; i < HD; i += 64) {
        kv.k8[row * HD + i] = static_cast<int8_t>(fmaxf(-127.0f, fminf(127.0f, rintf(kr[i] * ik))));
        kv.v8[row * HD + i] = static_cast<int8_t>(fmaxf(-127.0f, fminf(127.0f, rintf(vr[i] * iv))));
    }
}

// engine.cpp:1025-1039: attention residual, Hadamard MLP, mHC residual
// routing (hroute, whose Sinkhorn ran beside the attention) and lane mixing,
// the layer's hidden state; then the next
// layer's rms of x when `next_rms`. Thread i < D owns column i of every
// vector (loaded once at the start); only the Hadamard transforms go through
// LDS.
// With nxs (LDS, N * D floats, may alias mlp) the next layer's rms goes there
// instead of to b.nx; x[0..N) ends as thread i's column of the new lanes.
// after_loads() runs once the kernel's own loads are issued, before their
// first use (loads it issues are waited for after them).
template <int N, int WAVES, class F>
__device__ __forceinline__ void post_layer(const EngineBufs &b, const LayerDev &ld, int l,
                                           int next_rms, const EngineDims &d, float *red, float *mlp, float *hr,
                                           float *hpo, float *nxs, float (&x)[8], F &&after_loads, float *xo,
                                           bool lead) {
    const int D = d.D, i = threadIdx.x;
    const bool own = i < D;
    // every load of the kernel, issued before the first wait (threads past D read zeros)
    float proj, gn = load_or_zero(ld.post_norm, D, i);
    if (d.ogroups > 0) {  // the out-projection's group terms (OutProj), added in group order as the GEMV does
        constexpr int kMaxParts = 8;
        float part[kMaxParts];
#pragma unroll
        for (int g = 0; g < kMaxParts; ++g) part[g] = load_or_zero(b.oparts + g * D, g < d.ogroups ? D : 0, i);
        proj = 0.0f;
#pragma unroll
        for (int g = 0; g < kMaxParts; ++g)
            if (g < d.ogroups) proj += part[g];
    } else {
        proj = load_or_zero(b.proj, D, i);
    }
    float bx = load_or_zero(b.bx, D, i), u = load_or_zero(b.u, D, i);
    const float gh = load_or_zero(ld.pre_hada, D, i), d1 = load_or_zero(ld.d1, D, i);
    const float d3 = load_or_zero(ld.d3, D, i);
#pragma unroll
    for (int n = 0; n < N; ++n) x[n] = load_or_zero(b.x + n * D, D, i);
    const float d2 = load_or_zero(ld.d2, d.hada, i);
    // residual routing (computed beside the attention), used by wave 0
    const int lane = threadIdx.x & 63;
    const float route = load_or_zero(b.hroute, N * N, lane), hpost = load_or_zero(b.hpost, N, lane);
    after_loads();
    const float ag = sigmoidf_(ld.attn_gate[0]);
    if (threadIdx.x < 64) {
        if (lane < N * N) hr[lane] = route;
        if (lane < N) hpo[lane] = hpost;
    }
    // proj = rms(proj) * (1 + post_norm); bx += sigmoid(attn_gate) * proj
    // (red holds 2 * WAVES floats: the block sums alternate between its halves)
    float r = 1.0f / sqrtf(block_sum_nb(own ? proj * proj : 0.0f, red) / static_cast<float>(D) + 1e-6f);
    proj = proj * r * (1.0f + gn);
    bx += ag * proj;
    // z = rms(bx) * (1 + pre_hada); mlp = hadamard(silu_diag(hadamard(z * d1 | 0), d2)) (engine.cpp:1029-1033)
    r = 1.0f / sqrtf(block_sum_nb(own ? bx * bx : 0.0f, red + WAVES) / static_cast<float>(D) + 1e-6f);
    const float z = bx * r * (1.0f + gh);
    float mv;  // value i of the MLP vector (own threads)
    if (d.hada == 64 * WAVES) {  // one value per thread: the transforms in registers, mlp as staging
        const float a = hadamard_thread<WAVES>(own ? z * d1 : 0.0f, mlp, d.inv_hada) * d2;
        mv = hadamard_thread<WAVES>(a * sigmoidf_(a), mlp + d.hada, d.inv_hada);
    } else {
        if (i < d.hada) mlp[i] = own ? z * d1 : 0.0f;  // columns past D are zero padding (D <= threads)
        for (int k = i + blockDim.x; k < d.hada; k += blockDim.x) mlp[k] = 0.0f;
        __syncthreads();
        hadamard_block(mlp, d.hada, d.inv_hada);
        for (int k = threadIdx.x; k < d.hada; k += blockDim.x) {
            const float a = mlp[k] * (k == i ? d2 : ld.d2[k]);
            mlp[k] = a * sigmoidf_(a);
        }
        __syncthreads();
        hadamard_block(mlp, d.hada, d.inv_hada);
        mv = own ? mlp[i] : 0.0f;
    }
    // bx = bx + d3 * mlp - u; x[n] = hpost[n] bx + sum_j hres[n][j] x[j]; hidden = mean over lanes
    float ss = 0.0f;
    if (own) {
        bx = bx + d3 * mv - u;
        float nx[8], sum = 0.0f;
#pragma unroll
        for (int n = 0; n < N; ++n) {
            float val = hpo[n] * bx;
#pragma unroll
            for (int j = 0; j < N; ++j) val += hr[n * N + j] * x[j];
            nx[n] = val;
        }
#pragma unroll
        for (int n = 0; n < N; ++n) {
            if (lead) xo[n * D + i] = nx[n];
            sum += nx[n];
            ss += nx[n] * nx[n];
            x[n] = nx[n];
        }
        if (lead) b.hidden[l * D + i] = sum / static_cast<float>(N);
    }
    if (next_rms) {  // the next layer's nx = rms(x) over all N * D values
        r = 1.0f / sqrtf(block_sum_nb(ss, red) / static_cast<float>(N * D) + 1e-6f);
        float *nx = nxs ? nxs : b.nx;
        if (own)
#pragma unroll
            for (int n = 0; n < N; ++n) nx[n * D + i] = x[n] * r;
    }
}

// final_norm set (the last layer): then zf = rms(hidden) * (1 + final_norm) (engine.cpp:1041-1042), thread i
// holding hidden value i.
template <int N>
__global__ __launch_bounds__(kEngThreads) void eng_post_kernel(EngineBufs b0, LayerDev ld, int l, int next_rms,
                                                               EngineDims d, const float *__restrict__ final_norm) {
    const EngineBufs b = at_token(b0, d, blockIdx.y);
    __shared__ float red[2 * (kEngThreads / 64)];
    __shared__ float mlp[4096];
    __shared__ float hr[64], hpo[8];
    float x[8];
    post_layer<N, kEngThreads / 64>(b, ld, l, next_rms, d, red, mlp, hr, hpo, nullptr, x, [] {}, b.x, true);
    if (final_norm) {
        const int i = threadIdx.x;
        const bool own = i < d.D;
        const float h = own ? b.hidden[l * d.D + i] : 0.0f;  // this thread's own store above
        const float gain = own ? final_norm[i] : 0.0f;
        const float r = 1.0f / sqrtf(block_sum(h * h, red) / static_cast<float>(d.D) + 1e-6f);
        if (own) b.zf[i] = h * r * (1.0f + gain);
    }
}

__global__ __launch_bounds__(kEngThreads) void eng_quantize_kernel(float *x, int n, int stride, int bits) {
    __shared__ float red[kEngThreads / 64];
    quantize_block(x + static_cast<size_t>(blockIdx.y) * stride, n, bits, red);
}

// One wave per output row of a dense fp32 matrix.
__global__ __launch_bounds__(256) void eng_dense_kernel(const float *__restrict__ w, int cols, int first, int rows,
                                                        const float *__restrict__ x, float *__restrict__ y,
                                                        int ystride) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    x += static_cast<size_t>(blockIdx.y) * cols;
    y += static_cast<size_t>(blockIdx.y) * ystride;
    const float *row = w + static_cast<size_t>(first + r) * cols;
    float s = 0.0f;
    for (int i = lane; i < cols; i += 64) s += row[i] * x[i];
    s = wave_sum(s, lane);
    if (lane == 0) y[r] = s;
}

// Rows of up to three dense matrices over one input, one workgroup per row:
// block b < rows[0] is row first[0] + b of w[0] into y[0][b], and so on.
struct DenseRows {
    const float *w[3];
    float *y[3];
    int first[3], rows[3];
};

__global__ __launch_bounds__(256) void eng_dense_multi_kernel(DenseRows a, int cols, int ystride,
                                                              const float *__restrict__ x) {
    __shared__ float red[4];
    x += static_cast<size_t>(blockIdx.y) * cols;
    int r = blockIdx.x, m = 0;
    while (m < 2 && r >= a.rows[m]) r -= a.rows[m++];
    const float *row = a.w[m] + static_cast<size_t>(a.first[m] + r) * cols;
    float s = 0.0f;
    for (int i = threadIdx.x; i < cols; i += blockDim.x) s += row[i] * x[i];
    s = block_sum(s, red);
    if (threadIdx.x == 0) a.y[m][static_cast<size_t>(blockIdx.y) * ystride + r] = s;
}

// Row r of the dense mHC projections: pre rows, then post rows, then res rows.
__device__ __forceinline__ const float4 *mhc_row_ptr(const DenseRows &w, int r, int N, int cols) {
    const int m = r < N ? 0 : r < 2 * N ? 1 : 2;
    const int local = r - (m == 0 ? 0 : m == 1 ? N : 2 * N);
    const float *base = m == 0 ? w.w[0] : m == 1 ? w.w[1] : w.w[2];
    const int first = m == 0 ? w.first[0] : m == 1 ? w.first[1] : w.first[2];
    return reinterpret_cast<const float4 *>(base + static_cast<size_t>(first + local) * cols);
}

// One workgroup per token does eng_post_kernel's work for layer l, then the
// next layer's dense mHC projections (eng_dense_multi_kernel's rows) and
// eng_mix_kernel's work (engine.cpp:1024-1040, then 968-992 of layer l + 1),
// which saves two launches per layer. The projection weights (rows of N * D
// floats, N * D a multiple of 256) are loaded at the start, into registers,
// while the post waits on its own loads; the rms'd lanes stay in LDS and each
// thread's column of the new lanes in registers. One wave sums a projection
// row in eng_dense_multi_kernel's order: lane l's float4 column l + 64 k holds
// element k of that kernel's threads 4 l .. 4 l + 3, whose partial sums the
// lane keeps apart, and block_sum's tree over 64 threads and the sequential
// sum of its four waves follow, so the outputs are the same bits as the
// separate launches'. Needs D <= THREADS, N * D <= 4096.
// QKVG (one token, THREADS 512, no activation quantiser, no
// int8 target): workgroup blockIdx.x also computes one kQkvgRows-row slice of the
// next layer's Q|K|V|gate projection (QkvgFused); workgroup 0 alone stores
// the layer state, the lanes, u, bx and hpost into qf's *_out buffers.
// START: no post; the token's lanes come from its embedding row ez (eng_start_kernel's work), then layer
// 0's projections and mixing (l is -1).
template <int THREADS, int N, bool QKVG, bool START>
__global__ __launch_bounds__(THREADS) void eng_post_mix_kernel(EngineBufs b0, LayerDev ld, LayerDev ldn, MhcDev mh,
                                                               int l, DenseRows w, MixArgs m, EngineDims d,
                                                               PrepTarget pt, QkvgFused qf, const float *ez,
                                                               EmbedRows er) {
    struct Args {
        EngineBufs b0;
        LayerDev ld, ldn;
        MhcDev mh;
        int l;
        DenseRows w;
        MixArgs m;
        EngineDims d;
        PrepTarget pt;
        QkvgFused qf;
        const float *ez;
        EmbedRows er;
    };
    static_assert(!QKVG || THREADS == 512, "the fused projection takes 4 threads per row of its slice");
    touch_kernargs<QKVG ? offsetof(Args, ez) : offsetof(Args, pt)>();
    constexpr int kWaves = THREADS / 64, kPF = 8;  // float4 columns per lane held for each prefetched row
    constexpr int R = 2 * N + N * N;              // mHC projection rows
    constexpr int kRowsPF = std::min((R + kWaves - 1) / kWaves, 3);  // rows per wave held in registers
    const EngineBufs b = at_token(b0, d, blockIdx.y);
    __shared__ float red[2 * kWaves];
    __shared__ float mlp[4096];  // the MLP vector, then the rms'd lanes
    __shared__ float hr[64], hpo[8], hp[16];
    __shared__ float zs[QKVG ? 1 : 4096], ps[QKVG ? 1 : 4096];
    __shared__ float proj[2 * 8 + 64];
    // the projection's product table (4-bit: 17-float slot per position; 2-bit: 36-float slot per pair of
    // positions) and the parked group terms of groups 1 .. 3
    __shared__ __attribute__((aligned(16))) float tab[QKVG ? 256 * 36 : 1];
    __shared__ float park[QKVG ? 3 * kQkvgRows : 1];
    const int D = d.D, cols = N * D, c4n = cols / 4;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63, i = threadIdx.x;
    const bool lead = !QKVG || blockIdx.x == 0;
    // QKVG: this thread's row r of the workgroup's slice and group g, its codes (4 chunks of 4-bit codes or
    // 2 of 2-bit) and half norm, requested after the post's own loads and the projection-row prefetch (the
    // waits for those, counted in issue order, then do not wait for these; rows past the piece and groups
    // past the input: zeros)
    const int qr = i % kQkvgRows, qg = i / kQkvgRows;
    u32x4 qc[4];
    uint32_t qn = 0;
    float *qy = nullptr;
    int qrow = 0, qrows = 0;
    __amdgpu_buffer_rsrc_t qrc = buffer_rsrc(qf.piece[0].codes, 0u), qrn = buffer_rsrc(qf.piece[0].norms, 0u);
    uint32_t qtile = 0, qrr = 0, qlive = 0;
    if constexpr (QKVG) {
        const int wg = blockIdx.x;
        int pi = 0;
#pragma unroll
        for (int k = 1; k < 4; ++k)
            if (k < qf.pieces && wg >= qf.piece[k].sub_begin) pi = k;
        auto pick = [&](auto get) {  // piece pi's field without indexing the argument block at run time
            auto v = get(qf.piece[0]);
#pragma unroll
            for (int k = 1; k < 4; ++k)
                if (pi == k) v = get(qf.piece[k]);
            return v;
        };
        const uint4 *codes = pick([](const QkvgPiece &p) { return p.codes; });
        const uint16_t *norms = pick([](const QkvgPiece &p) { return p.norms; });
        qy = pick([](const QkvgPiece &p) { return p.y; });
        qrows = pick([](const QkvgPiece &p) { return p.rows; });
        const int sub = wg - pick([](const QkvgPiece &p) { return p.sub_begin; });
        qrow = sub * kQkvgRows + qr;
        const uint32_t tiles = static_cast<uint32_t>((qrows + 255) / 256);
        qrc = buffer_rsrc(codes, __builtin_amdgcn_readfirstlane(tiles * static_cast<uint32_t>(qf.chunks) * 4096u));
        qrn = buffer_rsrc(norms, __builtin_amdgcn_readfirstlane(tiles * static_cast<uint32_t>(qf.groups) * 512u));
        qtile = static_cast<uint32_t>(qrow >> 8);
        qrr = static_cast<uint32_t>(qrow & 255);
        qlive = qrow < qrows && qg < qf.groups ? 0u : 0x40000000u;  // else past the resource
    }
    float4 pf[kRowsPF][kPF];
    float x[8];
    GateParams gp;
    float nin;
    auto issue = [&] {
        // buffer loads over each row (wave-uniform): a row past R and columns
        // past the row read zero, so no load waits behind a branch
#pragma unroll
        for (int j = 0; j < kRowsPF; ++j) {
            const int r = wave + j * kWaves;
            const __amdgpu_buffer_rsrc_t rs =
                buffer_rsrc(mhc_row_ptr(w, r < R ? r : 0, N, cols), r < R ? static_cast<uint32_t>(c4n) * 16u : 0u);
#pragma unroll
            for (int k = 0; k < kPF; ++k)
                pf[j][k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                          rs, static_cast<uint32_t>(lane + 64 * k) * 16u, 0, 0));
        }
        gp = gate_params<N>(mh, l + 1);
        nin = load_or_zero(ldn.norm_in, D, i);
        if constexpr (QKVG) {
            const int cpg = qf.kind == 0 ? 4 : 2;  // code chunks per group of 128 positions
#pragma unroll
            for (int c = 0; c < 4; ++c)
                qc[c] = __builtin_amdgcn_raw_buffer_load_b128(
                    qrc, (c < cpg ? qlive : 0x40000000u) |
                             (((qtile * qf.chunks + static_cast<uint32_t>(qg * cpg + c)) * 256u + qrr) * 16u), 0, 0);
            qn = __builtin_amdgcn_raw_buffer_load_b16(
                qrn, qlive | (((qtile * qf.groups + static_cast<uint32_t>(qg)) * 256u + qrr) * 2u), 0, 0);
        }
    };
    float *const xo = QKVG ? qf.x_out : b.x;
    if constexpr (START) {
        // the token's lanes x[n] = embedding * sqrt(d_model) and their rms (engine.cpp:972-974), the rms'd
        // lanes into LDS for the projections below (l is -1: layer 0's mixing follows)
        float ze;
        if (er.codes) {  // the token's embedding row: cb[code] * half(norm) at position i, then the FWHT
            const CqGeom &g = er.g;
            const int row = static_cast<int>(er.ids[blockIdx.y]);
            const int own_i = i < D ? i : 0;
            const int cpc = g.kind == kNib ? 32 : 64, c = own_i / cpc, within = own_i % cpc;
            const uint4 v = er.codes[code_index(row, c, g.chunks)];
            const uint32_t words[4] = {v.x, v.y, v.z, v.w};
            const uint32_t code = g.kind == kNib ? (words[within >> 3] >> ((within & 7) * 4)) & 15u
                                                 : (words[within >> 4] >> ((within & 15) * 2)) & 3u;
            const float norm = h2f(er.norms[norm_index(row, own_i / g.group, g.groups)]);
            issue();
            ze = i < D ? g.lut[code] * norm : 0.0f;
            // stages h = 1 .. group / 2 in order, (a + b, a - b) as the transform kernel's
            if (g.group > 1) ze = fwht_stage<1>(ze, lane);
            if (g.group > 2) ze = fwht_stage<2>(ze, lane);
            if (g.group > 4) ze = fwht_stage<4>(ze, lane);
            if (g.group > 8) ze = fwht_stage<8>(ze, lane);
            if (g.group > 16) ze = fwht_stage<16>(ze, lane);
            if (g.group > 32) ze = fwht_stage<32>(ze, lane);
            for (int h = 64; h < g.group; h <<= 1) {
                mlp[i] = ze;
                __syncthreads();
                const float o = mlp[i ^ h];
                __syncthreads();
                ze = (i & h) ? o - ze : ze + o;
            }
            ze = i < D ? ze * g.scale : 0.0f;
            if (lead && i < D) er.z[static_cast<size_t>(blockIdx.y) * D + i] = ze;
        } else {
            ze = load_or_zero(ez + static_cast<size_t>(blockIdx.y) * D, D, i);
            issue();
        }
        float ss = 0.0f;
#pragma unroll
        for (int n = 0; n < N; ++n) {
            x[n] = ze * d.sqrt_d;
            ss += x[n] * x[n];
        }
        const float r = 1.0f / sqrtf(block_sum_nb(ss, red) / static_cast<float>(N * D) + 1e-6f);
        if (i < D)
#pragma unroll
            for (int n = 0; n < N; ++n) {
                mlp[n * D + i] = x[n] * r;
                if (lead) xo[n * D + i] = x[n];
            }
    } else {
        post_layer<N, kWaves>(b, ld, l, 1, d, red, mlp, hr, hpo, mlp, x, issue, xo, lead);
    }
    __syncthreads();
    const float4 *nx4 = reinterpret_cast<const float4 *>(mlp);
    auto fma4 = [](float4 &acc, const float4 &a, const float4 &c) {
        acc.x += a.x * c.x;
        acc.y += a.y * c.y;
        acc.z += a.z * c.z;
        acc.w += a.w * c.w;
    };
    auto row_sum = [&](float4 acc) {  // threads 4 lane .. 4 lane + 3 -> block_sum over 256 threads
        float v = (acc.x + acc.y) + (acc.z + acc.w);
        v += butterfly_partner<1>(v, lane);
        v += butterfly_partner<2>(v, lane);
        v += butterfly_partner<4>(v, lane);
        v += butterfly_partner<8>(v, lane);
        const int iv = __builtin_bit_cast(int, v);
        float total = 0.0f;
        total += __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
        total += __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
        total += __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
        total += __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
        return total;
    };
    float4 nxr[kPF];  // the lane's first columns of the rms'd lanes, for every row
#pragma unroll
    for (int k = 0; k < kPF; ++k) nxr[k] = lane + 64 * k < c4n ? nx4[lane + 64 * k] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < kRowsPF; ++j) {
        const int r = wave + j * kWaves;  // uniform over the wave
        if (r < R) {
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int k = 0; k < kPF; ++k)
                if (lane + 64 * k < c4n) fma4(acc, pf[j][k], nxr[k]);
            const float4 *row = mhc_row_ptr(w, r, N, cols);
            for (int c = lane + 64 * kPF; c < c4n; c += 64) fma4(acc, row[c], nx4[c]);
            const float sum = row_sum(acc);
            if (lane == 0) proj[r] = sum;
        }
    }
    for (int r = wave + kRowsPF * kWaves; r < R; r += kWaves) {
        const float4 *row = mhc_row_ptr(w, r, N, cols);
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int c = lane; c < c4n; c += 64) fma4(acc, row[c], nx4[c]);
        const float sum = row_sum(acc);
        if (lane == 0) proj[r] = sum;
    }
    __syncthreads();
    mix_gates<N>(b, gp, l + 1, proj, hp, QKVG ? qf.hpost_out : b.hpost, lead);
    __syncthreads();
    const bool own = i < D;
    float u = 0.0f;
    if (own) {
#pragma unroll
        for (int n = 0; n < N; ++n) u += hp[n] * x[n];
        if (lead) {
            (QKVG ? qf.u_out : b.u)[i] = u;
            (QKVG ? qf.bx_out : b.bx)[i] = u;
        }
    }
    float z = 0.0f;  // this thread's z after the quantiser (own threads)
    if (!QKVG && m.nsites) {
        __syncthreads();
        mix_sites(b, m, d, red, zs, ps);
        rms_block(b.bx, b.z, D, ldn.norm_in, red);
    } else if (QKVG && m.nsites) {
        // mix_sites' and rms_block's arithmetic on the registers (thread i holds element i), so that every
        // workgroup holds the same z; workgroup 0 stores bx
        float bxv = u;
        for (int k = 0; k < m.nsites; ++k) {
            int st = m.sites[0];
#pragma unroll
            for (int j = 1; j < kEngMaxSites; ++j)
                if (k == j) st = m.sites[j];
            const float ek = own ? b.ek[st * D + i] : 0.0f, ev = own ? b.ev[st * D + i] : 0.0f;
            const float ru = 1.0f / sqrtf(block_sum(own ? u * u : 0.0f, red) / static_cast<float>(D) + 1e-6f);
            const float rk = 1.0f / sqrtf(block_sum(own ? ek * ek : 0.0f, red) / static_cast<float>(D) + 1e-6f);
            const float zsv = u * ru, psv = ek * rk;
            const float alpha = sigmoidf_(block_sum(own ? zsv * psv : 0.0f, red) / d.sqrt_d);
            bxv = bxv + alpha * ev;
        }
        if (lead && own) qf.bx_out[i] = bxv;
        const float r = 1.0f / sqrtf(block_sum(own ? bxv * bxv : 0.0f, red) / static_cast<float>(D) + 1e-6f);
        if (own) {
            z = bxv * r * (1.0f + nin);
            if (lead) b.z[i] = z;
        }
        __syncthreads();
    } else {  // rms_block's arithmetic on the registers
        const float r = 1.0f / sqrtf(block_sum_nb(own ? u * u : 0.0f, red + kWaves) / static_cast<float>(D) + 1e-6f);
        if (own) {
            z = u * r * (1.0f + nin);
            if (lead) b.z[i] = z;
        }
        __syncthreads();
    }
    if constexpr (!QKVG) {
        quantize_block(b.z, D, d.abits, red);
        if (pt.q) {  // the next Q|K|V|gate projection's int8 input, from z staged in LDS
            if (own) zs[i] = m.nsites || d.abits ? b.z[i] : z;
            __syncthreads();
            prepare_groups(pt, zs, 0, D, 0, pt.dev / pt.group, 0, blockIdx.y, gridDim.y);
        }
    } else {
        // the GEMV's in-kernel FWHT of each group of 128 positions (thread i: position i; stages 1 .. 32 in
        // the wave, 64 through LDS; the same butterflies and operands), then * 1 / sqrt(128)
        float xr = own ? z : 0.0f;
        wave_butterflies<128, 1>(xr, lane);
        mlp[i] = xr;  // free: the rms'd lanes were last read before the mixing barriers
        __syncthreads();
        const float o = mlp[i ^ 64];
        xr = o + ((i & 64) ? -xr : xr);
        xr = xr * qf.scale;
        // the product table (the GEMV kernels' layout): 4-bit, slot p = position p, entry c = cb[c] * rot_p at a
        // 17-float stride; 2-bit, slot s = positions 2s, 2s + 1, entry c0 | c1 << 2 = (cb[c0] * rot_2s,
        // cb[c1] * rot_2s+1) at a 36-float stride
        if (qf.kind == 0) {
            if (own)
#pragma unroll
                for (int c = 0; c < 16; ++c) tab[i * 17 + c] = qf.lut[c] * xr;
        } else {
            const int pl = lane & 31;
            const float r0 = __shfl(xr, 2 * pl), r1 = __shfl(xr, 2 * pl + 1);
            if (own && lane < 32) {
                float p0[4], p1[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    p0[c] = qf.lut[c] * r0;
                    p1[c] = qf.lut[c] * r1;
                }
                float4 *dst = reinterpret_cast<float4 *>(tab + ((i & ~63) / 2 + pl) * 36);
#pragma unroll
                for (int hi = 0; hi < 4; ++hi) {
                    dst[2 * hi] = make_float4(p0[0], p1[hi], p0[1], p1[hi]);
                    dst[2 * hi + 1] = make_float4(p0[2], p1[hi], p0[3], p1[hi]);
                }
            }
        }
        __syncthreads();
        // row qr's group qg: gd over the group's 128 positions in order, times the half norm
        float gd = 0.0f;
        if (qf.kind == 0) {
            const float *tg = tab + (qg & 3) * 128 * 17;  // (threads past the groups read a group's slots)
#pragma unroll
            for (int dw = 0; dw < 16; ++dw) {
                const uint32_t cw = qc[dw >> 2][dw & 3];
#pragma unroll
                for (int k = 0; k < 8; ++k) gd += tg[(8 * dw + k) * 17 + ((cw >> (4 * k)) & 15u)];
            }
        } else {
            const float *tg = tab + (qg & 3) * 64 * 36;
#pragma unroll
            for (int dw = 0; dw < 8; ++dw) {
                const uint32_t cw = qc[dw >> 2][dw & 3];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float2 e = *reinterpret_cast<const float2 *>(tg + (8 * dw + k) * 36 + 2 * ((cw >> (4 * k)) & 15u));
                    gd += e.x;
                    gd += e.y;
                }
            }
        }
        const float pg = gd * h2f(static_cast<uint16_t>(qn));
        if (qg > 0 && qg < 4) park[(qg - 1) * kQkvgRows + qr] = pg;
        __syncthreads();
        if (qg == 0) {  // the row sum in group order
            float sum = 0.0f;
            sum += pg;
#pragma unroll
            for (int k = 1; k < 4; ++k)
                if (k < qf.groups) sum += park[(k - 1) * kQkvgRows + qr];
            if (qrow < qrows) qy[qrow] = sum;
        }
    }
}

__global__ __launch_bounds__(256) void eng_dense_rows_kernel(const float *__restrict__ w, int cols,
                                                             const int64_t *__restrict__ ids, int count,
                                                             float *__restrict__ y) {
    const int i = blockIdx.y;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += gridDim.x * blockDim.x)
        y[static_cast<size_t>(i) * cols + c] = w[static_cast<size_t>(ids[i]) * cols + c];
}

}  // namespace

// f(std::integral_constant<int, N>) for the engine's lane count N (1, 2, 4 or 8).
template <class F>
void with_lanes(int n, F &&f) {
    switch (n) {
    case 1: f(std::integral_constant<int, 1>{}); break;
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    default: f(std::integral_constant<int, 8>{}); break;
    }
}

void launch_eng_start(const float *z, const EngineBufs &b, const EngineDims &d, int tokens, hipStream_t s) {
    hipLaunchKernelGGL(eng_start_kernel, dim3(1, tokens), dim3(kEngThreads), 0, s, z, b, d);
    ND_HIP(hipGetLastError());
}

void launch_eng_engram_in(const EngineBufs &b, const StepParams *p, int site, const EngineDims &d, int tokens,
                          hipStream_t s) {
    hipLaunchKernelGGL(eng_engram_in_kernel, dim3(1, tokens), dim3(kEngThreads), 0, s, b, p, site, d);
    ND_HIP(hipGetLastError());
}

void launch_eng_engram_out(const EngineBufs &b, const float *taps, const StepParams *p, int site,
                           const EngineDims &d, int tokens, hipStream_t s) {
    hipLaunchKernelGGL(eng_engram_conv_kernel, dim3(1, tokens), dim3(kEngThreads), 0, s, b, taps, p, site, d);
    ND_HIP(hipGetLastError());
    hipLaunchKernelGGL(eng_engram_ring_kernel, dim3(1, std::min(tokens, d.engring)), dim3(kEngThreads), 0, s, b, p,
                       site, tokens, d);
    ND_HIP(hipGetLastError());
}

void launch_eng_mix(const EngineBufs &b, const LayerDev &ld, const MhcDev &mh, int l, const int *mhc_row,
                    const int *sites, int nsites, const EngineDims &d, int tokens, const PrepTarget &pt,
                    hipStream_t s) {
    MixArgs m{};
    m.l = l;
    m.nsites = nsites;
    for (int i = 0; i < nsites; ++i) m.sites[i] = sites[i];
    for (int i = 0; i < 3; ++i) m.mhc_row[i] = mhc_row[i];
    with_lanes(d.N, [&](auto n) {
        hipLaunchKernelGGL(eng_mix_kernel<decltype(n)::value>, dim3(1, tokens), dim3(kEngThreads), 0, s, b, ld, mh, m,
                           d, pt);
    });
    ND_HIP(hipGetLastError());
}

void launch_eng_qk(const EngineBufs &b, const LayerDev &ld, const KvLayer &kv, const StepParams *p,
                   const EngineDims &d, int tokens, hipStream_t s) {
    hipLaunchKernelGGL(eng_qk_kernel, dim3(1, tokens), dim3(kEngThreads), 0, s, b, ld, kv, p, d);
    ND_HIP(hipGetLastError());
}

void launch_eng_attn_fused(const EngineBufs &b, const LayerDev &ld, const KvLayer &kv, const StepParams *p,
                           const StepParams &hp, int max_length, bool prepared, const EngineDims &d, int tokens,
                           float *scores, size_t scores_n, const MhcDev &mh, int l, const PrepTarget &pt,
                           const OutProj &op, hipStream_t s) {
    const StepHead sh{hp.slot, hp.length, hp.prefix_count, hp.start, hp.prefix, hp.window, hp.ring};
    ND_CHECK(!op.codes || (d.H / d.KV * d.HD == 128 && !pt.q && op.rows <= 512 && d.KV <= 8),
             "internal: fused out-projection outside its geometry");
    // the score slices are [tokens][kv heads][G][max_length] (the routing workgroup touches none)
    ND_CHECK(!scores || static_cast<size_t>(tokens) * d.KV * (d.H / d.KV) * static_cast<size_t>(max_length) <= scores_n,
             "internal: attention score buffer smaller than tokens * kv heads * G * max_length");
    ND_CHECK(!pt.q || (pt.group == d.H / d.KV * d.HD && pt.group <= 256 && pt.dev == d.A),
             "internal: attention prepares one kv head's outputs as one group");
    const size_t lds = scores ? 0 : static_cast<size_t>(d.H / d.KV) * max_length * sizeof(float);
    ND_CHECK(lds <= kEngScoreLds, "internal: attention scores exceed the LDS budget without a score buffer");
    OutProj o = op;  // several workgroups per kv head only for one token with the scores in LDS
    if (scores || tokens != 1 || !o.codes) o.split_shift = 0;
    ND_CHECK(o.split_shift >= 0 && o.split_shift <= 2, "internal: out-projection split outside 1, 2 or 4");
    const dim3 grid((d.KV << o.split_shift) + 1, tokens), block(256);  // the last workgroup: the routing
    const bool wide = d.HD > 128 || d.H / d.KV + 1 > 4;  // the norms' one-head-per-wave form needs neither
    auto go = [&](auto i8) {
        constexpr bool I8 = decltype(i8)::value;
        if (prepared && scores)
            hipLaunchKernelGGL((eng_attn_fused_kernel<true, true, I8>), grid, block, 0, s, b, ld, kv, p, sh, d, scores,
                               max_length, mh, l, pt, o);
        else if (prepared)
            hipLaunchKernelGGL((eng_attn_fused_kernel<true, false, I8>), grid, block, lds, s, b, ld, kv, p, sh, d, nullptr,
                               0, mh, l, pt, o);
        else if (wide && scores)
            hipLaunchKernelGGL((eng_attn_fused_kernel<false, true, I8, true>), grid, block, 0, s, b, ld, kv, p, sh, d,
                               scores, max_length, mh, l, pt, o);
        else if (wide)
            hipLaunchKernelGGL((eng_attn_fused_kernel<false, false, I8, true>), grid, block, lds, s, b, ld, kv, p, sh, d,
                               nullptr, 0, mh, l, pt, o);
        else if (scores)
            hipLaunchKernelGGL((eng_attn_fused_kernel<false, true, I8>), grid, block, 0, s, b, ld, kv, p, sh, d, scores,
                               max_length, mh, l, pt, o);
        else
            hipLaunchKernelGGL((eng_attn_fused_kernel<false, false, I8>), grid, block, lds, s, b, ld, kv, p, sh, d,
                               nullptr, 0, mh, l, pt, o);
    };
    if (kv.k8) go(std::true_type{});
    else go(std::false_type{});
    ND_HIP(hipGetLastError());
}

void launch_eng_kv_import(const float *k, const float *v, const int *slots, int count, const KvLayer &kv,
                          const EngineDims &d, hipStream_t s) {
    if (count <= 0) return;
    hipLaunchKernelGGL(eng_kv_import_kernel, dim3(count * d.KV), dim3(64), 0, s, k, v, slots, kv, d);
    ND_HIP(hipGetLastError());
}

void launch_eng_post(const EngineBufs &b, const LayerDev &ld, int l, bool next_rms,
                     const EngineDims &d, int tokens, const float *final_norm, hipStream_t s) {
    ND_CHECK(!final_norm || (l == d.layers - 1 && !next_rms && d.D <= kEngThreads),
             "internal: the final norm follows the last layer's post");
    with_lanes(d.N, [&](auto n) {
        hipLaunchKernelGGL(eng_post_kernel<decltype(n)::value>, dim3(1, tokens), dim3(kEngThreads), 0, s, b, ld, l,
                           next_rms ? 1 : 0, d, final_norm);
    });
    ND_HIP(hipGetLastError());
}

bool eng_post_mix_fits(const EngineDims &d) {
    return d.D <= kEngThreads && d.N * d.D <= 4096 && (d.N * d.D) % 256 == 0 && d.hada <= 4096;
}

void launch_eng_post_mix(const EngineBufs &b, const LayerDev &ld, const LayerDev &ldn, const MhcDev &mh, int l,
                         const float *const *w, const int *first, const int *sites, int nsites, const EngineDims &d,
                         int tokens, const PrepTarget &pt, const QkvgFused *qf, const float *start, hipStream_t s,
                         const EmbedRows &er) {
    ND_CHECK(eng_post_mix_fits(d), "internal: fused post / mixing launch outside its geometry");
    ND_CHECK(!qf || (tokens == 1 && !pt.q && d.abits == 0 && d.D <= 512 && d.D % 128 == 0 &&
                     qf->wgs > 0 && qf->pieces >= 1 && qf->pieces <= 4 && qf->groups == d.D / 128 &&
                     (qf->kind == 0 || qf->kind == 1) && qf->x_out && qf->u_out && qf->bx_out && qf->hpost_out),
             "internal: fused Q|K|V|gate projection outside its geometry");
    DenseRows a{};
    for (int k = 0; k < 3; ++k) {
        a.w[k] = w[k];
        a.first[k] = first[k];
    }
    MixArgs m{};
    m.l = l + 1;
    m.nsites = nsites;
    for (int k = 0; k < nsites; ++k) m.sites[k] = sites[k];
    ND_CHECK(!start || l == -1, "internal: the first layer's mixing takes l = -1");
    ND_CHECK(!er.codes || (start && d.D <= 512 && er.g.group <= d.D && er.g.groups * er.g.group == d.D &&
                           (er.g.kind == kNib || er.g.kind == kCrumb)),
             "internal: embedding rows decoded in the first launch outside its geometry");
    const QkvgFused none{};
    auto go = [&](auto n, auto st) {
        constexpr int N = decltype(n)::value;
        constexpr bool S = decltype(st)::value;
        if (qf)
            hipLaunchKernelGGL((eng_post_mix_kernel<512, N, true, S>), dim3(qf->wgs, 1), dim3(512), 0, s, b, ld, ldn,
                               mh, l, a, m, d, pt, *qf, start, er);
        else if (d.D <= 512)
            hipLaunchKernelGGL((eng_post_mix_kernel<512, N, false, S>), dim3(1, tokens), dim3(512), 0, s, b, ld, ldn,
                               mh, l, a, m, d, pt, none, start, er);
        else
            hipLaunchKernelGGL((eng_post_mix_kernel<kEngThreads, N, false, S>), dim3(1, tokens), dim3(kEngThreads), 0,
                               s, b, ld, ldn, mh, l, a, m, d, pt, none, start, EmbedRows{});
    };
    with_lanes(d.N, [&](auto n) {
        if (start) go(n, std::true_type{});
        else go(n, std::false_type{});
    });
    ND_HIP(hipGetLastError());
}

void launch_eng_quantize(float *x, int n, int stride, int bits, int tokens, hipStream_t s) {
    if (!bits) return;
    hipLaunchKernelGGL(eng_quantize_kernel, dim3(1, tokens), dim3(kEngThreads), 0, s, x, n, stride, bits);
    ND_HIP(hipGetLastError());
}

void launch_eng_dense(const float *w, int cols, int first, int rows, const float *x, float *y, int ystride,
                      int tokens, hipStream_t s) {
    if (rows <= 0) return;
    hipLaunchKernelGGL(eng_dense_kernel, dim3((rows + 3) / 4, tokens), dim3(256), 0, s, w, cols, first, rows, x, y,
                       ystride);
    ND_HIP(hipGetLastError());
}

void launch_eng_dense3(const float *const *w, const int *first, const int *rows, float *const *y, int ystride,
                       int cols, const float *x, int tokens, hipStream_t s) {
    DenseRows a{};
    int total = 0;
    for (int m = 0; m < 3; ++m) {
        a.w[m] = w[m];
        a.y[m] = y[m];
        a.first[m] = first[m];
        a.rows[m] = w[m] ? rows[m] : 0;
        total += a.rows[m];
    }
    if (!total) return;
    hipLaunchKernelGGL(eng_dense_multi_kernel, dim3(total, tokens), dim3(256), 0, s, a, cols, ystride, x);
    ND_HIP(hipGetLastError());
}

void launch_eng_dense_rows(const float *w, int cols, const int64_t *ids, int count, float *y, hipStream_t s) {
    if (count <= 0) return;
    hipLaunchKernelGGL(eng_dense_rows_kernel, dim3((cols + 255) / 256, count), dim3(256), 0, s, w, cols, ids, count,
                       y);
    ND_HIP(hipGetLastError());
}

}  // namespace nd
