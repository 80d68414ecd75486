// C ABI of the int8 KV cache and batched decode attention (additive exports).
//
// The reference keeps the int8 cache inside its Engine (engine.cpp:433-449
// allocation, 1005-1021 quantize/store, 898-967 compute_attention) and
// exposes it only through needle2_engine_set_int8_kv / _kv_storage_bytes.
// This library exposes the same arithmetic as a device-resident cache for
// many sequences at once: store quantizes new K/V rows, attention runs one
// decode step for every sequence of one layer.
#include "abi_internal.h"
#include "attn.h"

#include <algorithm>
#include <cmath>
#include <memory>
#include <vector>

namespace nd {

struct KvHandle {
    int layers = 0, capacity = 0, kvheads = 0, head_dim = 0, seqs = 0;
    DevBuf<int8_t> k8, v8;
    DevBuf<float> ks, vs;
    DevBuf<float> part;
    DevBuf<int> first;    // per-sequence first slot of a store
    HostBuf<int> hfirst;  // pinned staging for `first`
    hipEvent_t first_copied = nullptr;

    size_t layer_codes() const { return size_t(seqs) * kvheads * capacity * head_dim; }
    size_t layer_scales() const { return size_t(seqs) * kvheads * capacity; }
    ~KvHandle() {
        if (first_copied) (void)hipEventDestroy(first_copied);
    }
};

static KvHandle *kv_of(void *h) {
    ND_CHECK(h != nullptr, "null KV cache handle");
    return static_cast<KvHandle *>(h);
}

static void check_layer(const KvHandle &kv, int layer) {
    ND_CHECK(layer >= 0 && layer < kv.layers, "KV cache: layer out of range");
}

// Splits of the slot range: enough (sequence, kv head, split) blocks for two
// per CU, never a split shorter than one 256-slot tile. With that many
// (sequence, kv head) pairs already (a large decode batch) there is one split
// and no merge pass.
static int auto_splits(int pairs, int length) {
    static const int cus = [] {  // queried once
        int dev = 0, n = 256;
        if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        return n;
    }();
    const int tiles = (length + 255) / 256;
    const int want = (2 * cus + pairs - 1) / pairs;
    return std::max(1, std::min(want, tiles));
}

}  // namespace nd

using namespace nd;

extern "C" {

// Device cache of `layers` x `seqs` sequences x `capacity` slots x `kvheads`
// rows of `head_dim` int8 codes plus one fp32 scale per row, for K and V.
// Zero-filled (reference reset, engine.cpp:433-449). NULL + needle2_gpu_error()
// on failure.
void *needle2_gpu_kv_create(int layers, int capacity, int kvheads, int head_dim, int seqs) {
    KvHandle *kv = nullptr;
    if (guarded([&] {
            ND_CHECK(layers > 0 && capacity > 0 && kvheads > 0 && seqs > 0, "KV cache: sizes must be positive");
            ND_CHECK(head_dim == 32 || head_dim == 64 || head_dim == 128, "KV cache: head_dim must be 32, 64 or 128");
            ND_CHECK(size_t(capacity) * head_dim < (size_t(1) << 31), "KV cache: capacity * head_dim must be < 2^31");
            auto h = std::make_unique<KvHandle>();
            h->layers = layers;
            h->capacity = capacity;
            h->kvheads = kvheads;
            h->head_dim = head_dim;
            h->seqs = seqs;
            const size_t nc = h->layer_codes() * layers, ns = h->layer_scales() * layers;
            h->k8.reserve(nc);
            h->v8.reserve(nc);
            h->ks.reserve(ns);
            h->vs.reserve(ns);
            ND_HIP(hipMemset(h->k8.p, 0, nc));
            ND_HIP(hipMemset(h->v8.p, 0, nc));
            ND_HIP(hipMemset(h->ks.p, 0, ns * sizeof(float)));
            ND_HIP(hipMemset(h->vs.p, 0, ns * sizeof(float)));
            h->first.reserve(seqs);
            h->hfirst.reserve(seqs);
            ND_HIP(hipEventCreateWithFlags(&h->first_copied, hipEventDisableTiming));
            ND_HIP(hipEventRecord(h->first_copied, nullptr));
            ND_HIP(hipDeviceSynchronize());
            kv = h.release();
        }))
        return nullptr;
    return kv;
}

void needle2_gpu_kv_destroy(void *kv) { delete static_cast<KvHandle *>(kv); }

// Bytes of cache storage (codes + scales), as needle2_engine_kv_storage_bytes
// reports for the int8 cache (engine.cpp:433-449).
size_t needle2_gpu_kv_storage_bytes(void *h) {
    if (!h) return 0;
    const KvHandle &kv = *static_cast<KvHandle *>(h);
    return (kv.layer_codes() * 2 + kv.layer_scales() * 2 * sizeof(float)) * kv.layers;
}

// Quantize and store `count` new tokens per sequence into `layer`.
// d_k, d_v: device fp32 [seqs][count][kvheads][head_dim] (keys after RoPE, as
// the reference stores them). Token i of sequence s goes to slot
// seq_first_slot[s] + i (host array, nullable: first_slot for every sequence).
int needle2_gpu_kv_store(void *h, int layer, const float *d_k, const float *d_v, int count, int first_slot,
                         const int *seq_first_slot, void *stream) {
    return guarded([&] {
        KvHandle &kv = *kv_of(h);
        check_layer(kv, layer);
        ND_CHECK(count >= 0, "KV store: count must be >= 0");
        if (count == 0) return;
        ND_CHECK(d_k && d_v, "KV store: null input");
        hipStream_t s = static_cast<hipStream_t>(stream);
        ND_HIP(hipEventSynchronize(kv.first_copied));  // the previous store's upload has finished
        for (int i = 0; i < kv.seqs; ++i) {
            const int f = seq_first_slot ? seq_first_slot[i] : first_slot;
            ND_CHECK(f >= 0 && f + count <= kv.capacity, "KV store: slots outside the cache capacity");
            kv.hfirst.p[i] = f;
        }
        ND_HIP(hipMemcpyAsync(kv.first.p, kv.hfirst.p, kv.seqs * sizeof(int), hipMemcpyHostToDevice, s));
        ND_HIP(hipEventRecord(kv.first_copied, s));
        KvStoreArgs a{};
        a.k = d_k;
        a.v = d_v;
        a.k8 = kv.k8.p + kv.layer_codes() * layer;
        a.v8 = kv.v8.p + kv.layer_codes() * layer;
        a.ks = kv.ks.p + kv.layer_scales() * layer;
        a.vs = kv.vs.p + kv.layer_scales() * layer;
        a.first_slot = kv.first.p;
        a.seqs = kv.seqs;
        a.count = count;
        a.kvheads = kv.kvheads;
        a.head_dim = kv.head_dim;
        a.capacity = kv.capacity;
        launch_kv_store(a, s);
    });
}

// needle2_gpu_kv_store with the per-sequence first slots already in device
// memory (d_first_slot[seqs]): no host copy and no host wait, so a decode
// step built from it can be captured in a HIP graph and replayed while the
// caller advances d_first_slot on the device. Rows whose slot falls outside
// [0, capacity) are skipped.
int needle2_gpu_kv_store_device(void *h, int layer, const float *d_k, const float *d_v, int count,
                                const int *d_first_slot, void *stream) {
    return guarded([&] {
        KvHandle &kv = *kv_of(h);
        check_layer(kv, layer);
        ND_CHECK(count >= 0, "KV store: count must be >= 0");
        if (count == 0) return;
        ND_CHECK(d_k && d_v && d_first_slot, "KV store: null input");
        KvStoreArgs a{};
        a.k = d_k;
        a.v = d_v;
        a.k8 = kv.k8.p + kv.layer_codes() * layer;
        a.v8 = kv.v8.p + kv.layer_codes() * layer;
        a.ks = kv.ks.p + kv.layer_scales() * layer;
        a.vs = kv.vs.p + kv.layer_scales() * layer;
        a.first_slot = d_first_slot;
        a.seqs = kv.seqs;
        a.count = count;
        a.kvheads = kv.kvheads;
        a.head_dim = kv.head_dim;
        a.capacity = kv.capacity;
        launch_kv_store(a, static_cast<hipStream_t>(stream));
    });
}

// One decode-attention step (needle2_gpu_attention below), optionally with
// the step's new token and the next projection:
// - d_new_k, d_new_v, d_new_slot (all or none; device [seqs][kvheads]
//   [head_dim] fp32 and [seqs] slots): first stores that token of every
//   sequence at its slot, as needle2_gpu_kv_store_device with count 1 - in
//   the attention launch without a slot list (by the block whose split
//   holds the slot), else by the store launch before it;
// - next (a one-matrix int8 plan of batch seqs whose input buffer is d_out,
//   e.g. the O projection): d_out is also left prepared as next's input, for
//   needle2_gpu_plan_run_chained(next, ..., prepared = 1) - in the
//   attention's epilogue for groups of 32 and one split, else by next's
//   prepare launch (not at all when next's GEMV prepares its own input).
int needle2_gpu_attention_chained(void *h, int layer, const float *d_q, float *d_out, int heads, int length,
                                  const int *d_slots, const int *d_lengths, int splits, const float *d_new_k,
                                  const float *d_new_v, const int *d_new_slot, void *next, void *stream) {
    return guarded([&] {
        KvHandle &kv = *kv_of(h);
        check_layer(kv, layer);
        ND_CHECK(heads > 0 && heads % kv.kvheads == 0, "attention: heads must be a multiple of kvheads");
        const int group = heads / kv.kvheads;
        ND_CHECK(attn_supported(kv.head_dim, group), "attention: query heads per kv head must be 1, 2, 4 or 8");
        ND_CHECK(length >= 0 && (d_slots || length <= kv.capacity), "attention: length exceeds the cache capacity");
        ND_CHECK(d_q && d_out, "attention: null q or out");
        hipStream_t s = static_cast<hipStream_t>(stream);
        const int pairs = kv.seqs * kv.kvheads;
        if (splits <= 0) splits = auto_splits(pairs, length);
        const int tiles = std::max(1, (length + 255) / 256);
        splits = std::min(splits, tiles);
        const int per = (tiles + splits - 1) / splits * 256;  // whole tiles per split
        splits = std::max(1, (length + per - 1) / per);
        AttnArgs a{};
        a.k8 = kv.k8.p + kv.layer_codes() * layer;
        a.v8 = kv.v8.p + kv.layer_codes() * layer;
        a.ks = kv.ks.p + kv.layer_scales() * layer;
        a.vs = kv.vs.p + kv.layer_scales() * layer;
        a.q = d_q;
        a.out = d_out;
        if (splits > 1) kv.part.reserve(size_t(kv.seqs) * heads * splits * (kv.head_dim + 2));
        a.part = kv.part.p;
        a.slots = d_slots;
        a.lengths = d_lengths;
        a.seqs = kv.seqs;
        a.kvheads = kv.kvheads;
        a.head_dim = kv.head_dim;
        a.capacity = kv.capacity;
        a.length = length;
        a.splits = splits;
        a.slots_per_split = per;
        a.scale = 1 / std::sqrt(float(kv.head_dim));  // engine.cpp:914
        ND_CHECK(!d_new_k == !d_new_v && !d_new_k == !d_new_slot, "attention: new K, V and slots come together");
        if (d_new_k) {
            if (!d_slots) {
                a.new_k = d_new_k;
                a.new_v = d_new_v;
                a.new_slot = d_new_slot;
            } else {
                KvStoreArgs st{};
                st.k = d_new_k;
                st.v = d_new_v;
                st.k8 = kv.k8.p + kv.layer_codes() * layer;
                st.v8 = kv.v8.p + kv.layer_codes() * layer;
                st.ks = kv.ks.p + kv.layer_scales() * layer;
                st.vs = kv.vs.p + kv.layer_scales() * layer;
                st.first_slot = d_new_slot;
                st.seqs = kv.seqs;
                st.count = 1;
                st.kvheads = kv.kvheads;
                st.head_dim = kv.head_dim;
                st.capacity = kv.capacity;
                launch_kv_store(st, s);
            }
        }
        const PrepOut po = plan_prep_target(next, d_out, heads * kv.head_dim, kv.seqs);
        const bool feed = next && plan_wants_input(next);  // not when next's GEMV prepares its own input
        const bool fused = feed && po.q && splits == 1 && group * kv.head_dim % 64 == 0;
        if (fused) a.prep = po;
        launch_attention(a, group, s);
        if (fused) plan_mark_staged(next);
        else if (feed) plan_prepare_input(next, s);
    });
}

// One decode-attention step of `layer` for every sequence.
// d_q, d_out: device fp32 [seqs][heads][head_dim]; heads is a multiple of
// kvheads (1, 2, 4 or 8 query heads per kv head). Sequence s attends the
// slots d_slots[j] (device, at least `length` entries, nullable: j) for
// j < d_lengths[s] (device, nullable: length); no sequence attends more than
// `length` slots, and a listed slot outside [0, capacity) is skipped.
// splits: pieces the slot range is cut into (0: chosen from the device).
int needle2_gpu_attention(void *h, int layer, const float *d_q, float *d_out, int heads, int length,
                          const int *d_slots, const int *d_lengths, int splits, void *stream) {
    return needle2_gpu_attention_chained(h, layer, d_q, d_out, heads, length, d_slots, d_lengths, splits, nullptr,
                                         nullptr, nullptr, nullptr, stream);
}

// Copy host rows in the reference's layout ([count][kvheads][head_dim] int8,
// [count][kvheads] fp32 scales) into slots [first_slot, first_slot + count)
// of one sequence and layer (synchronous).
int needle2_gpu_kv_import(void *h, int layer, int seq, const int8_t *k, const int8_t *v, const float *ks,
                          const float *vs, int first_slot, int count) {
    return guarded([&] {
        KvHandle &kv = *kv_of(h);
        check_layer(kv, layer);
        ND_CHECK(seq >= 0 && seq < kv.seqs, "KV import: sequence out of range");
        ND_CHECK(first_slot >= 0 && count >= 0 && first_slot + count <= kv.capacity, "KV import: slots out of range");
        const int HD = kv.head_dim, KV = kv.kvheads;
        for (int kh = 0; kh < KV; ++kh) {
            const size_t row = (size_t(seq) * KV + kh) * kv.capacity + first_slot;
            int8_t *dk = kv.k8.p + kv.layer_codes() * layer + row * HD;
            int8_t *dv = kv.v8.p + kv.layer_codes() * layer + row * HD;
            ND_HIP(hipMemcpy2D(dk, HD, k + size_t(kh) * HD, size_t(KV) * HD, HD, count, hipMemcpyHostToDevice));
            ND_HIP(hipMemcpy2D(dv, HD, v + size_t(kh) * HD, size_t(KV) * HD, HD, count, hipMemcpyHostToDevice));
            float *dks = kv.ks.p + kv.layer_scales() * layer + row;
            float *dvs = kv.vs.p + kv.layer_scales() * layer + row;
            ND_HIP(hipMemcpy2D(dks, sizeof(float), ks + kh, size_t(KV) * sizeof(float), sizeof(float), count,
                               hipMemcpyHostToDevice));
            ND_HIP(hipMemcpy2D(dvs, sizeof(float), vs + kh, size_t(KV) * sizeof(float), sizeof(float), count,
                               hipMemcpyHostToDevice));
        }
    });
}

// Inverse of needle2_gpu_kv_import (synchronous).
int needle2_gpu_kv_export(void *h, int layer, int seq, int8_t *k, int8_t *v, float *ks, float *vs, int first_slot,
                          int count) {
    return guarded([&] {
        KvHandle &kv = *kv_of(h);
        check_layer(kv, layer);
        ND_CHECK(seq >= 0 && seq < kv.seqs, "KV export: sequence out of range");
        ND_CHECK(first_slot >= 0 && count >= 0 && first_slot + count <= kv.capacity, "KV export: slots out of range");
        ND_HIP(hipDeviceSynchronize());
        const int HD = kv.head_dim, KV = kv.kvheads;
        for (int kh = 0; kh < KV; ++kh) {
            const size_t row = (size_t(seq) * KV + kh) * kv.capacity + first_slot;
            const int8_t *sk = kv.k8.p + kv.layer_codes() * layer + row * HD;
            const int8_t *sv = kv.v8.p + kv.layer_codes() * layer + row * HD;
            ND_HIP(hipMemcpy2D(k + size_t(kh) * HD, size_t(KV) * HD, sk, HD, HD, count, hipMemcpyDeviceToHost));
            ND_HIP(hipMemcpy2D(v + size_t(kh) * HD, size_t(KV) * HD, sv, HD, HD, count, hipMemcpyDeviceToHost));
            const float *sks = kv.ks.p + kv.layer_scales() * layer + row;
            const float *svs = kv.vs.p + kv.layer_scales() * layer + row;
            ND_HIP(hipMemcpy2D(ks + kh, size_t(KV) * sizeof(float), sks, sizeof(float), sizeof(float), count,
                               hipMemcpyDeviceToHost));
            ND_HIP(hipMemcpy2D(vs + kh, size_t(KV) * sizeof(float), svs, sizeof(float), sizeof(float), count,
                               hipMemcpyDeviceToHost));
        }
    });
}

}  // extern "C"
