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
// The dot runs over d in the reference's order but with fused multiply-adds
// (one rounding per term instead of two), and the value sums likewise. The
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
#include "sdot_prepare.h"
#include "wave.h"

#include <cmath>

namespace nd {

namespace {

// One K row and one V row of HD values into the cache, by one wave.
__device__ __forceinline__ void store_kv_row(const float *k, const float *v, int HD, int lane, int8_t *k8, int8_t *v8,
                                             float *ks, float *vs) {
    float mk = 0.0f, mv = 0.0f;
    for (int d = lane; d < HD; d += 64) {
        mk = fmaxf(mk, fabsf(k[d]));
        mv = fmaxf(mv, fabsf(v[d]));
    }
    mk = wave_max(mk, lane);
    mv = wave_max(mv, lane);
    const float sk = mk > 0 ? mk / 127.0f : 1.0f, sv = mv > 0 ? mv / 127.0f : 1.0f;
    const float ik = mk > 0 ? 127.0f / mk : 0.0f, iv = mv > 0 ? 127.0f / mv : 0.0f;
    if (lane == 0) {
        *ks = sk;
        *vs = sv;
    }
    for (int d = lane; d < HD; d += 64) {
        float qk = rintf(k[d] * ik), qv = rintf(v[d] * iv);
        qk = fmaxf(-127.0f, fminf(127.0f, qk));
        qv = fmaxf(-127.0f, fminf(127.0f, qv));
        k8[d] = static_cast<int8_t>(qk);
        v8[d] = static_cast<int8_t>(qv);
    }
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
    const int slot = a.first_slot[seq] + i;
    if (slot < 0 || slot >= a.capacity) return;  // wave-uniform; device-side slot tables are not host-checked
    const size_t src = static_cast<size_t>(wave) * a.head_dim;
    const size_t dst_row = (static_cast<size_t>(seq) * a.kvheads + kh) * a.capacity + slot;
    const int HD = a.head_dim;
    store_kv_row(a.k + src, a.v + src, HD, lane, a.k8 + dst_row * HD, a.v8 + dst_row * HD, a.ks + dst_row,
                 a.vs + dst_row);
}

__device__ __forceinline__ float i8f(uint32_t w, int c) {
    return static_cast<float>(static_cast<int8_t>((w >> (8 * c)) & 0xffu));
}

// Block (split, kv head, sequence): 4 waves, each an independent
// online-softmax worker over 64-slot sub-tiles w, w + 4, w + 8, ... of the
// block's slot range, with the next sub-tile's loads in flight while the
// current one is computed. No block barrier inside the loop; the 4 waves'
// (m, l, o) are combined once at the end.
//   Score phase: lane = slot; the K row is HD/16 16-byte loads; q comes from
//   scalar loads (uniform); dot by fma over d.
//   Value phase: a slot row is HD/4 words, VW words per lane, LPR = HD/4/VW
//   lanes per row, 64/LPR slot lanes, LPR slots per lane per sub-tile.
// All cache reads are buffer loads over this context's rows: a slot that is
// not attended (past the range, or outside [0, capacity) in the caller's
// list) gets an offset past the buffer and reads zero without a memory
// request, so loads need no branches.
template <int HD, int G, int VW, bool SLOTS>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs a) {
    constexpr int DW = HD / 4;
    constexpr int LPR = DW / VW;   // lanes per value row
    constexpr int NLW = 64 / LPR;  // slot lanes per wave
    constexpr int SPL = LPR;       // slots per lane per sub-tile
    constexpr int KC = HD / 16;    // 16-byte chunks per K row
    constexpr uint32_t kOut = 0x80000000u;  // past every buffer (capacity * HD < 2^31)
    static_assert(DW % VW == 0 && 64 % LPR == 0, "value-phase lane mapping");
    __shared__ float lw[4][G][64];
    __shared__ float lred[4][NLW][G][HD];
    __shared__ float lm[4][G], ll[4][G];

    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int sp = blockIdx.x, kh = blockIdx.y, seq = blockIdx.z;
    const int H = a.kvheads * G;
    int len = a.lengths ? a.lengths[seq] : a.length;
    len = len < a.length ? len : a.length;
    const int begin = sp * a.slots_per_split;
    const int end = min(begin + a.slots_per_split, len);
    const uint32_t cap = static_cast<uint32_t>(a.capacity);

    const ND_CONST float *qh = (const ND_CONST float *)(a.q + (static_cast<size_t>(seq) * H + kh * G) * HD);
    const size_t row0 = (static_cast<size_t>(a.shared_cache ? 0 : seq) * a.kvheads + kh) * cap;
    const auto rk = buffer_rsrc(a.k8 + row0 * HD, cap * HD);
    const auto rv = buffer_rsrc(a.v8 + row0 * HD, cap * HD);
    const auto rks = buffer_rsrc(a.ks + row0, cap * 4u);
    const auto rvs = buffer_rsrc(a.vs + row0, cap * 4u);
    const auto rsl = buffer_rsrc(a.slots + static_cast<size_t>(seq) * a.slots_stride, static_cast<uint32_t>(a.length) * 4u);
    const int vj = lane % LPR, vr = lane / LPR;  // value phase: word group, slot lane

    // slot of list position s, or -1 when not attended
    auto slot_of = [&](int s) -> int {
        int raw = s;
        if constexpr (SLOTS) raw = static_cast<int>(__builtin_amdgcn_raw_buffer_load_b32(rsl, s * 4u, 0, 0));
        return (s < end && static_cast<uint32_t>(raw) < cap) ? raw : -1;
    };

    struct Tile {
        u32x4 k[KC];
        uint32_t v[SPL][VW];
        float ks, vs;
        bool valid;
    };
    auto load = [&](Tile &T, int st) {
        const int slot = slot_of(st + lane);
        T.valid = slot >= 0;
        const uint32_t kb = slot >= 0 ? static_cast<uint32_t>(slot) * HD : kOut;
        const uint32_t sb = slot >= 0 ? static_cast<uint32_t>(slot) * 4u : kOut;
#pragma unroll
        for (int c = 0; c < KC; ++c) T.k[c] = __builtin_amdgcn_raw_buffer_load_b128(rk, kb, c * 16, 0);
        T.ks = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rks, sb, 0, 0));
        T.vs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvs, sb, 0, 0));
#pragma unroll
        for (int i = 0; i < SPL; ++i) {
            const int sv = slot_of(st + vr + i * NLW);
            const uint32_t vb = sv >= 0 ? static_cast<uint32_t>(sv) * HD + vj * VW * 4u : kOut;
            if constexpr (VW == 4) {
                const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rv, vb, 0, 0);
                T.v[i][0] = w.x;
                T.v[i][1] = w.y;
                T.v[i][2] = w.z;
                T.v[i][3] = w.w;
            } else {
#pragma unroll
                for (int u = 0; u < VW; ++u) T.v[i][u] = __builtin_amdgcn_raw_buffer_load_b32(rv, vb, u * 4, 0);
            }
        }
    };

    float m[G], l[G], acc[G][4 * VW];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4 * VW; ++c) acc[g][c] = 0.0f;
    }

    auto compute = [&](const Tile &T) {
        float alpha[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float dot = 0.0f;
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                const uint32_t w4[4] = {T.k[c].x, T.k[c].y, T.k[c].z, T.k[c].w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int b = 0; b < 4; ++b) dot = __builtin_fmaf(qh[g * HD + c * 16 + j * 4 + b], i8f(w4[j], b), dot);
            }
            float x = dot * T.ks;
            x *= a.scale;
            x = T.valid ? x : -INFINITY;
            const float mn = fmaxf(m[g], wave_max(x, lane));
            alpha[g] = mn == -INFINITY ? 1.0f : expf(m[g] - mn);
            m[g] = mn;
            const float e = T.valid ? expf(x - mn) : 0.0f;
            l[g] = l[g] * alpha[g] + e;
            lw[wave][g][lane] = e * T.vs;
        }
        // LDS operations of one wave complete in order; the fences only stop
        // the compiler from moving the reads above the writes (and the next
        // sub-tile's writes above these reads).
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int c = 0; c < 4 * VW; ++c) acc[g][c] *= alpha[g];
#pragma unroll
        for (int i = 0; i < SPL; ++i) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float w = lw[wave][g][vr + i * NLW];
#pragma unroll
                for (int u = 0; u < VW; ++u)
#pragma unroll
                    for (int b = 0; b < 4; ++b) acc[g][u * 4 + b] = __builtin_fmaf(w, i8f(T.v[i][u], b), acc[g][u * 4 + b]);
            }
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
    };

    // With a new token (no slot list, so list position = slot), wave 0 of
    // the block whose split holds slot new_slot[seq] (the last split for a
    // slot past every range; no block for one outside the cache) first stores
    // the token's K and V rows there as kv_store_kernel does; the block
    // barrier (a workgroup-scope release and acquire) orders those stores
    // before the block's loads of that slot, and no other block reads it.
    // When the slot lies past the waves' first sub-tiles, those loads are
    // issued before the store.
    auto store_new = [&](int ns) {
        if (wave == 0) {
            const size_t src = (static_cast<size_t>(seq) * a.kvheads + kh) * HD;
            const size_t dst = row0 + ns;
            store_kv_row(a.new_k + src, a.new_v + src, HD, lane, a.k8 + dst * HD, a.v8 + dst * HD, a.ks + dst,
                         a.vs + dst);
        }
        __syncthreads();
    };
    const int ns = a.new_k ? a.new_slot[seq] : -1;
    const bool store_here =
        a.new_k && ns >= 0 && static_cast<uint32_t>(ns) < cap && sp == min(ns / a.slots_per_split, a.splits - 1);
    const bool store_early = store_here && ns < begin + 256;  // the slot may be in a first sub-tile

    // The next sub-tile is loaded before this one is computed; loads past the
    // end read zero.
    Tile cur, nxt;
    int st = begin + wave * 64;
    if (store_early) store_new(ns);
    load(cur, st);
    if (store_here && !store_early) store_new(ns);
    for (; st < end; st += 256) {
        load(nxt, st + 256);
        asm volatile("" ::: "memory");  // keep the prefetch ahead of the compute
        compute(cur);
        cur = nxt;
    }
    // wave partials -> LDS; combine the 4 waves with their own maxima
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float ws = wave_sum(l[g], lane);
        if (lane == 0) {
            lm[wave][g] = m[g];
            ll[wave][g] = ws;
        }
#pragma unroll
        for (int c = 0; c < 4 * VW; ++c) lred[wave][vr][g][vj * 4 * VW + c] = acc[g][c];
    }
    __syncthreads();
    for (int i = t; i < G * HD; i += 256) {
        const int g = i / HD, d = i % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, lm[w][g]);
        float o = 0.0f, lt = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if (lm[w][g] == -INFINITY) continue;  // a wave with nothing attended
            const float f = expf(lm[w][g] - M);
            float ow = 0.0f;
            for (int r = 0; r < NLW; ++r) ow += lred[w][r][g][d];
            o += f * ow;
            lt += f * ll[w][g];
        }
        const size_t head = static_cast<size_t>(seq) * H + kh * G + g;
        if (a.splits == 1) {
            const float val = lt > 0 ? o * (1.0f / lt) : 0.0f;
            a.out[head * HD + d] = val;
            if (a.prep.q) {
                // whole waves (G * HD is a multiple of 64) over consecutive positions of the sequence's
                // output row: groups of 32 lanes are groups of the next projection's input
                const PrepOut &po = a.prep;
                const int p = (kh * G + g) * HD + d;
                prepare_lane<32>(val, lane, p, po.padded, po.dev, po.scale, po.kind,
                                 po.q + static_cast<size_t>(seq) * po.dev, po.xs + static_cast<size_t>(seq) * po.groups + p / 32,
                                 po.xst + static_cast<size_t>(p / 32) * po.batch + seq);
            }
        } else {
            float *rec = a.part + (head * a.splits + sp) * (HD + 2);
            rec[2 + d] = o;
            if (d == 0) {
                rec[0] = M;
                rec[1] = lt;
            }
        }
    }
}

// One block per query head: out = sum_i exp(m_i - M) o_i / sum_i exp(m_i - M) l_i, in split order.
// The records are read kMergeBatch splits at a time, every load of a batch in
// flight together (buffer loads with the whole offset in the range-checked
// lane offset: splits past the count read zero and are skipped), so a merge
// costs one memory round trip per batch, not per split.
constexpr int kMergeBatch = 16;
__global__ __launch_bounds__(128) void attn_merge_kernel(const float *__restrict__ part, float *__restrict__ out,
                                                         int heads_total, int splits, int hd) {
    const int head = blockIdx.x;
    const uint32_t stride = static_cast<uint32_t>(hd + 2) * 4u;  // bytes per split record
    const auto rr = buffer_rsrc(part + static_cast<size_t>(head) * splits * (hd + 2), static_cast<uint32_t>(splits) * stride);
    auto load = [&](int i, int field) {  // field 0: m, 1: l, 2 + d: o[d]
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             rr, static_cast<uint32_t>(i) * stride + static_cast<uint32_t>(field) * 4u, 0, 0));
    };
    float M = -INFINITY;
    for (int i0 = 0; i0 < splits; i0 += kMergeBatch) {
        float m[kMergeBatch];
#pragma unroll
        for (int k = 0; k < kMergeBatch; ++k) m[k] = load(i0 + k, 0);
#pragma unroll
        for (int k = 0; k < kMergeBatch; ++k)
            if (i0 + k < splits) M = fmaxf(M, m[k]);
    }
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float L = 0.0f, O = 0.0f;
        for (int i0 = 0; i0 < splits; i0 += kMergeBatch) {
            float m[kMergeBatch], l[kMergeBatch], o[kMergeBatch];
#pragma unroll
            for (int k = 0; k < kMergeBatch; ++k) {
                m[k] = load(i0 + k, 0);
                l[k] = load(i0 + k, 1);
                o[k] = load(i0 + k, 2 + d);
            }
#pragma unroll
            for (int k = 0; k < kMergeBatch; ++k) {
                if (i0 + k >= splits || m[k] == -INFINITY) continue;  // past the count, or an empty split
                const float f = expf(m[k] - M);
                L += f * l[k];
                O += f * o[k];
            }
        }
        out[static_cast<size_t>(head) * hd + d] = L > 0 ? O * (1.0f / L) : 0.0f;
    }
}

// 16-byte value loads (VW = 4) while the accumulators fit; single words for
// 4 or 8 query heads per kv head.
template <int HD, bool SLOTS>
void launch_attn_hd(const AttnArgs &a, int G, dim3 grid, hipStream_t s) {
    switch (G) {
    case 1: hipLaunchKernelGGL((attn_kernel<HD, 1, 4, SLOTS>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attn_kernel<HD, 2, 4, SLOTS>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((attn_kernel<HD, 4, 1, SLOTS>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((attn_kernel<HD, 8, 1, SLOTS>), grid, dim3(256), 0, s, a); break;
    default: ND_CHECK(false, "attention: heads per kv head must be 1, 2, 4 or 8");
    }
    ND_HIP(hipGetLastError());
}

template <int HD>
void launch_attn_slots(const AttnArgs &a, int G, dim3 grid, hipStream_t s) {
    if (a.slots) launch_attn_hd<HD, true>(a, G, grid, s);
    else launch_attn_hd<HD, false>(a, G, grid, s);
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
    case 32: launch_attn_slots<32>(a, group, grid, s); break;
    case 64: launch_attn_slots<64>(a, group, grid, s); break;
    default: launch_attn_slots<128>(a, group, grid, s); break;
    }
    if (a.splits > 1) {
        hipLaunchKernelGGL(attn_merge_kernel, dim3(a.seqs * H), dim3(128), 0, s, a.part, a.out, a.seqs * H, a.splits,
                           a.head_dim);
        ND_HIP(hipGetLastError());
    }
}

}  // namespace nd
