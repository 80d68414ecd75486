// gfx950 kernels for the int8 KV cache: quantize/store and decode attention.
//
// Store (engine.cpp:1005-1021): per (token, kv head) row, max = absmax,
// scale = max > 0 ? max/127 : 1, inv = max > 0 ? 127/max : 0,
// q = clamp(rint(x * inv), +-127) - multiply by the reciprocal, IEEE
// division for scale and inv, so codes and scales are bit-identical.
//
// Attention (engine.cpp:898-967, 56-74, 137-147, 816-897): for each query
// head h of kv head kh = h / G,
//   s = dot(q_h, float(k_i8)) * k_scale * (1/sqrt(HD))   (sequential over d)
//   p = softmax(s);  out[d] = sum_s (p_s * v_scale_s) * float(v_i8[s][d]).
// The dot is the reference's sequential fp32 sum (no contraction). The
// softmax and the value sum are computed split-context (flash decoding):
// each block owns a range of cache slots for one (sequence, kv head) and
// keeps a running max m, a running sum l and unnormalized outputs o; a merge
// pass rescales by exp(m_i - M). That reorders fp32 sums, so results agree
// with the reference to fp32 rounding, not bit for bit.
//
// Device layout (head-major so one (sequence, kv head) context is one
// contiguous run): codes [layer][seq][kvh][capacity][HD] int8, scales
// [layer][seq][kvh][capacity] fp32.
#include "attn.h"

#include <cmath>

namespace nd {

namespace {

constexpr int kTile = 256;  // cache slots per block iteration (one per thread in the score phase)

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// One wave per (sequence, token, kv head) row; K and V rows together.
__global__ __launch_bounds__(256) void kv_store_kernel(KvStoreArgs a) {
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    const int rows = a.seqs * a.count * a.kvheads;
    if (wave >= rows) return;
    const int kh = wave % a.kvheads;
    const int i = (wave / a.kvheads) % a.count;
    const int seq = wave / (a.kvheads * a.count);
    const int slot = a.first_slot[seq] + i;  // validated on the host
    const size_t src = static_cast<size_t>(wave) * a.head_dim;
    const size_t dst_row = (static_cast<size_t>(seq) * a.kvheads + kh) * a.capacity + slot;
    const int HD = a.head_dim;
    float mk = 0.0f, mv = 0.0f;
    for (int d = lane; d < HD; d += 64) {
        mk = fmaxf(mk, fabsf(a.k[src + d]));
        mv = fmaxf(mv, fabsf(a.v[src + d]));
    }
    mk = wave_max(mk);
    mv = wave_max(mv);
    const float sk = mk > 0 ? mk / 127.0f : 1.0f, sv = mv > 0 ? mv / 127.0f : 1.0f;
    const float ik = mk > 0 ? 127.0f / mk : 0.0f, iv = mv > 0 ? 127.0f / mv : 0.0f;
    if (lane == 0) {
        a.ks[dst_row] = sk;
        a.vs[dst_row] = sv;
    }
    for (int d = lane; d < HD; d += 64) {
        float qk = rintf(a.k[src + d] * ik), qv = rintf(a.v[src + d] * iv);
        qk = fmaxf(-127.0f, fminf(127.0f, qk));
        qv = fmaxf(-127.0f, fminf(127.0f, qv));
        a.k8[dst_row * HD + d] = static_cast<int8_t>(qk);
        a.v8[dst_row * HD + d] = static_cast<int8_t>(qv);
    }
}

__device__ __forceinline__ float i8f(uint32_t w, int c) {
    return static_cast<float>(static_cast<int8_t>((w >> (8 * c)) & 0xffu));
}

// Block (split, kv head, sequence). HD: head dim; G: query heads per kv head.
template <int HD, int G>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
    constexpr int DW = HD / 4;        // int8x4 words per cache row
    constexpr int NL = kTile / DW;    // slot lanes in the value phase
    constexpr int TPT = kTile / NL;   // slots per thread per tile in the value phase (== DW)
    __shared__ float lq[G][HD];
    __shared__ float lw[G][kTile];      // p_s * v_scale_s of the tile
    __shared__ float red[8][G];         // per-wave partial max / sum
    __shared__ float lred[NL][G][HD];   // value-phase lane partials

    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int sp = blockIdx.x, kh = blockIdx.y, seq = blockIdx.z;
    const int H = a.kvheads * G;
    int len = a.lengths ? a.lengths[seq] : a.length;
    len = len < a.length ? len : a.length;
    const int begin = sp * a.slots_per_split;
    const int end = min(begin + a.slots_per_split, len);

    for (int i = t; i < G * HD; i += 256)
        lq[i / HD][i % HD] = a.q[(static_cast<size_t>(seq) * H + kh * G) * HD + i];
    const size_t row0 = (static_cast<size_t>(seq) * a.kvheads + kh) * a.capacity;
    const int8_t *kc = a.k8 + row0 * HD;
    const int8_t *vc = a.v8 + row0 * HD;
    const float *ksc = a.ks + row0;
    const float *vsc = a.vs + row0;
    __syncthreads();

    float m[G], l[G], acc[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
        acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0.0f;
    }
    const int vj = t % DW, vr = t / DW;  // value phase: word and slot lane

    for (int base = begin; base < end; base += kTile) {
        // issue the tile's K row (score phase) and V words (value phase) together
        // a slot outside [0, capacity) in the caller's list is not attended
        const int s = base + t;
        const int slot_raw = s < end ? (a.slots ? a.slots[s] : s) : -1;
        const bool valid = static_cast<unsigned>(slot_raw) < static_cast<unsigned>(a.capacity);
        const int slot = valid ? slot_raw : 0;
        u32x4 kr[HD / 16];
#pragma unroll
        for (int c = 0; c < HD / 16; ++c)
            kr[c] = valid ? reinterpret_cast<const u32x4 *>(kc + static_cast<size_t>(slot) * HD)[c] : u32x4{0, 0, 0, 0};
        const float kscale = valid ? ksc[slot] : 0.0f;
        const float vscale = valid ? vsc[slot] : 0.0f;
        uint32_t vw[TPT];
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            const int sv = base + vr + i * NL;
            const int slv = sv < end ? (a.slots ? a.slots[sv] : sv) : -1;
            vw[i] = static_cast<unsigned>(slv) < static_cast<unsigned>(a.capacity)
                        ? reinterpret_cast<const uint32_t *>(vc + static_cast<size_t>(slv) * HD)[vj]
                        : 0u;
        }
        // scores: the reference's sequential dot, then * k_scale, * 1/sqrt(HD)
        float sc[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float sum = 0.0f;
#pragma unroll
            for (int c = 0; c < HD / 16; ++c) {
                const uint32_t w4[4] = {kr[c].x, kr[c].y, kr[c].z, kr[c].w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int b = 0; b < 4; ++b) sum += lq[g][c * 16 + j * 4 + b] * i8f(w4[j], b);
            }
            float x = sum * kscale;
            x *= a.scale;
            sc[g] = valid ? x : -INFINITY;
        }
        // tile max -> running max
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float wm = wave_max(sc[g]);
            if (lane == 0) red[wave][g] = wm;
        }
        __syncthreads();
        float alpha[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float tm = red[0][g];
#pragma unroll
            for (int w = 1; w < 4; ++w) tm = fmaxf(tm, red[w][g]);
            const float mn = fmaxf(m[g], tm);
            alpha[g] = mn == -INFINITY ? 1.0f : expf(m[g] - mn);  // 0 on the first attended tile
            m[g] = mn;
            const float e = valid ? expf(sc[g] - mn) : 0.0f;
            l[g] = l[g] * alpha[g] + e;
            lw[g][t] = e * vscale;
        }
        __syncthreads();
        // value phase: acc[g][c] = alpha * acc + sum_i w_i * v_i[4 vj + c]
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[g][c] *= alpha[g];
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float w = lw[g][vr + i * NL];
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[g][c] = __builtin_fmaf(w, i8f(vw[i], c), acc[g][c]);
            }
        }
        __syncthreads();  // lw and red are rewritten by the next tile
    }
    // combine: l over all threads, acc over the NL slot lanes
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float ws = wave_sum(l[g]);
        if (lane == 0) red[wave][g] = ws;
#pragma unroll
        for (int c = 0; c < 4; ++c) lred[vr][g][vj * 4 + c] = acc[g][c];
    }
    __syncthreads();
    for (int i = t; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        float o = 0.0f;
        for (int r = 0; r < NL; ++r) o += lred[r][g][d];
        const float lt = red[0][g] + red[1][g] + red[2][g] + red[3][g];
        const size_t head = static_cast<size_t>(seq) * H + kh * G + g;
        if (a.splits == 1) {
            a.out[head * HD + d] = lt > 0 ? o * (1.0f / lt) : 0.0f;
        } else {
            float *rec = a.part + (head * a.splits + sp) * (HD + 2);
            rec[2 + d] = o;
            if (d == 0) {
                rec[0] = begin < end ? m[g] : -INFINITY;
                rec[1] = lt;
            }
        }
    }
}

// One block per query head: out = sum_i exp(m_i - M) o_i / sum_i exp(m_i - M) l_i.
__global__ __launch_bounds__(128) void attn_merge_kernel(const float *__restrict__ part, float *__restrict__ out,
                                                         int heads_total, int splits, int hd) {
    const int head = blockIdx.x;
    const float *rec = part + static_cast<size_t>(head) * splits * (hd + 2);
    float M = -INFINITY;
    for (int i = 0; i < splits; ++i) M = fmaxf(M, rec[i * (hd + 2)]);
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float L = 0.0f, O = 0.0f;
        for (int i = 0; i < splits; ++i) {
            const float mi = rec[i * (hd + 2)];
            if (mi == -INFINITY) continue;  // empty split
            const float f = expf(mi - M);
            L += f * rec[i * (hd + 2) + 1];
            O += f * rec[i * (hd + 2) + 2 + d];
        }
        out[static_cast<size_t>(head) * hd + d] = L > 0 ? O * (1.0f / L) : 0.0f;
    }
}

template <int HD>
void launch_attn_hd(const AttnArgs &a, int G, dim3 grid, hipStream_t s) {
    switch (G) {
    case 1: hipLaunchKernelGGL((attn_kernel<HD, 1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attn_kernel<HD, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((attn_kernel<HD, 4>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((attn_kernel<HD, 8>), grid, dim3(256), 0, s, a); break;
    default: ND_CHECK(false, "attention: heads per kv head must be 1, 2, 4 or 8");
    }
    ND_HIP(hipGetLastError());
}

}  // namespace

bool attn_supported(int head_dim, int group) {
    return (head_dim == 32 || head_dim == 64 || head_dim == 128) && (group == 1 || group == 2 || group == 4 || group == 8);
}

void launch_kv_store(const KvStoreArgs &a, hipStream_t s) {
    const int rows = a.seqs * a.count * a.kvheads;
    if (rows <= 0) return;
    hipLaunchKernelGGL(kv_store_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, a);
    ND_HIP(hipGetLastError());
}

void launch_attention(AttnArgs a, int group, hipStream_t s) {
    ND_CHECK(attn_supported(a.head_dim, group), "attention: unsupported head_dim / group");
    const int H = a.kvheads * group;
    dim3 grid(a.splits, a.kvheads, a.seqs);
    switch (a.head_dim) {
    case 32: launch_attn_hd<32>(a, group, grid, s); break;
    case 64: launch_attn_hd<64>(a, group, grid, s); break;
    default: launch_attn_hd<128>(a, group, grid, s); break;
    }
    if (a.splits > 1) {
        hipLaunchKernelGGL(attn_merge_kernel, dim3(a.seqs * H), dim3(128), 0, s, a.part, a.out, a.seqs * H, a.splits,
                           a.head_dim);
        ND_HIP(hipGetLastError());
    }
}

}  // namespace nd
