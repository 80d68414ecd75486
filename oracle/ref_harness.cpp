// Checker harness around the reference's own source (TEST INFRASTRUCTURE ONLY).
//
// oracle/Makefile compiles this file with -I pointing at the reference's
// needle2/csrc directory, so the translation unit below is the reference's
// cq.cpp (which itself includes sdot.cpp, engine.cpp and frontend.cpp) plus
// a few extern "C" entry points that reach code the reference's ABI does not
// expose on x86:
//   * SdotCQ: needle2_sdot_create returns NULL on x86 because runtime_dotprod()
//     is false (sdot.cpp:9-22, 352); its scalar branches are still compiled,
//     so the harness constructs SdotCQ directly.
//   * Engine::import_state (engine.cpp:784-815), whose int8 branch is the same
//     KV quantizer as Engine::step (engine.cpp:1005-1021), and
//     Engine::compute_attention (engine.cpp:898-967).
//   * Engine's SDOT matmul path: Engine::configure_sdot (engine.cpp:424-432)
//     returns false on x86 for the same reason, so refh_engine_sdot makes the
//     same SdotCQ matrices (2/4-bit codes, groups 64..131072) and switches
//     the path on, leaving every other line of the Engine as built.
// Output goes only to oracle/_ref/. No reference source is copied.
#include "cq.cpp"

extern "C" {

void *refh_sdot_create(const uint8_t *p, const uint16_t *n, int out, int in, int bits, int group, const float *cb) {
    try { return new SdotCQ(p, n, out, in, bits, group, cb); } catch (...) { return nullptr; }
}

void refh_sdot_destroy(void *h) { delete static_cast<SdotCQ *>(h); }

void refh_sdot_linear(void *h, const float *x, float *y, int batch, int threads) {
    auto *q = static_cast<SdotCQ *>(h);
    Prepared prep;
    for (int b = 0; b < batch; ++b) {
        q->prepare(x + size_t(b) * q->columns, prep);
        q->multiply(prep, y + size_t(b) * q->rows, threads);
    }
}

// Prepared activations in the reference's own (permuted) storage order.
void refh_sdot_prepare(void *h, const float *x, int8_t *q_out, float *scales_out) {
    auto *q = static_cast<SdotCQ *>(h);
    Prepared prep;
    q->prepare(x, prep);
    std::copy(prep.q.begin(), prep.q.end(), q_out);
    std::copy(prep.scales.begin(), prep.scales.end(), scales_out);
}

void refh_sdot_centroids(void *h, int8_t *centroids, float *centroid_scale, float *norm_scales) {
    auto *q = static_cast<SdotCQ *>(h);
    std::copy(q->centroids, q->centroids + (1 << q->bits), centroids);
    *centroid_scale = q->centroid_scale;
    std::copy(q->norm_scales.begin(), q->norm_scales.end(), norm_scales);
}

// One-layer engine holding only an int8 KV cache (no weights are touched by
// import_state / compute_attention when there are no Engram sites).
void *refh_attn_create(int heads, int kvheads, int head_dim, int max_seq, int threads) {
    try {
        EngineConfig c{};
        c.vocab = 1; c.dim = heads * head_dim; c.heads = heads; c.kvheads = kvheads;
        c.layers = 1; c.head_dim = head_dim; c.max_seq = max_seq; c.hada = 1; c.lanes = 1;
        c.window = 0; c.taps = 1; c.dilation = 1; c.rope_theta = 10000.0f;
        auto *e = new Engine(c, nullptr, 0, threads, 0);
        e->set_int8_kv(true);
        return e;
    } catch (...) { return nullptr; }
}

void refh_attn_destroy(void *e) { delete static_cast<Engine *>(e); }

// Quantize fp32 K/V rows [count][kvheads][head_dim] into cache positions 0..count-1.
int refh_attn_import(void *h, const float *k, const float *v, int count) {
    auto *e = static_cast<Engine *>(h);
    try {
        std::vector<int> ids(count > 0 ? count : 1, 0), positions(count > 0 ? count : 1);
        for (int i = 0; i < count; ++i) positions[i] = i;
        e->import_state(count, 0, ids.data(), positions.data(), count, k, v);
        return 0;
    } catch (...) { return -1; }
}

void refh_attn_cache(void *h, int8_t *keys, int8_t *values, float *k_scales, float *v_scales, int count) {
    auto *e = static_cast<Engine *>(h);
    size_t K = size_t(e->c.kvheads) * e->c.head_dim, KV = e->c.kvheads;
    std::copy(e->keys_i8.begin(), e->keys_i8.begin() + count * K, keys);
    std::copy(e->values_i8.begin(), e->values_i8.begin() + count * K, values);
    std::copy(e->k_scales.begin(), e->k_scales.begin() + count * KV, k_scales);
    std::copy(e->v_scales.begin(), e->v_scales.begin() + count * KV, v_scales);
}

// Attend query q [heads][head_dim] over positions 0..pos_cur of layer 0.
void refh_attn_compute(void *h, int pos_cur, const float *q, float *out) {
    static_cast<Engine *>(h)->compute_attention(0, pos_cur, q, out);
}

// engine.cpp:424-432 without the CPU feature test.
int refh_engine_sdot(void *h) {
    auto *e = static_cast<Engine *>(h);
    try {
        for (size_t i = 0; i < e->t.size(); ++i)
            if (e->t[i].cq) {
                auto *q = static_cast<CQ *>(e->t[i].cq);
                if ((q->bits == 2 || q->bits == 4) && q->group >= 64 && q->group <= 131072)
                    e->sdot[i] = std::make_unique<SdotCQ>(q->packed, q->norms, q->out, q->in, q->bits, q->group,
                                                          q->cb.data());
            }
        e->sdot_enabled = true;
        return 0;
    } catch (...) { return -1; }
}

}  // extern "C"
