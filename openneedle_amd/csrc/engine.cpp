// Single-sequence decode engine on the GPU behind the reference's
// needle2_engine_* ABI (needle2/csrc/engine.cpp:340-1044, 1499-1548;
// NativeEngine, needle2/native.py:307-663).
//
// One step (engine.cpp:968-1044) runs on the handle's stream as: embedding
// row, then per layer the mHC projections and the mixing kernel, the fused
// Q|K|V|gate GEMV, attention (fp32 KV: norms, RoPE, K / V store, attention
// and output gate in one launch; int8 KV: the norms + RoPE + store kernel,
// attention and the gate kernel; either launch also runs the layer's
// Sinkhorn routing in one more workgroup), the out-projection GEMV and the
// post kernel (attention residual, Hadamard MLP, lane mixing, next layer's
// rms), which for dense mHC matrices also runs the next layer's projections
// and mixing; then the final norm and the LM-head GEMV. The engram rows /
// projections / conv of each site depend on the token history only: they run
// on a second stream, which the step joins just before that site's mixing. The
// CQ matrices are the caller's handles (borrowed, as the reference borrows
// its CQ pointers) and run through the library's bit-exact GEMV kernels with
// the engine's own staging; dense tensors are copied to device memory at
// creation. The host computes what depends only on the position and the
// token history (slot lists, RoPE angles with std::cos / std::sin, engram
// hashes) and uploads it once per step.
#include "abi_internal.h"
#include "engine.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

namespace nd {

namespace {

// needle2/csrc/engine.cpp:14-19 (layouts must match the reference's).
struct TensorDescC {
    void *cq;
    const float *data;
    int rows, cols;
};
// needle2/csrc/engine.cpp:326-338: a compiled grammar as the decode loop reads it.
struct DfaC {
    int num_states, initial_state, eos_id, stop_id, tool_start_id, tool_end_id;
    const int *state_types;           // 0 open, 1 exact candidates, 4 terminal
    const int *fallback_next_states;  // -1: stay
    const int *candidate_offsets;     // [num_states + 1]
    const int *candidate_tokens;
    const int *next_states;
};

struct EngineConfigC {
    int vocab, dim, heads, kvheads, layers, head_dim, max_seq, hada, lanes, window;
    int slots, subdim, tables, taps, dilation, num_orders, orders[4], num_sites, sites[4];
    float rope_theta;
};

thread_local std::string engine_error;

// One matrix tensor of the model: a CQ handle or dense fp32 rows on the device.
struct Mat {
    const Matrix *cq = nullptr;
    const float *dense = nullptr;
    int rows = 0, cols = 0;
    bool int8 = false;  // the CQ matrix runs the int8 path (needle2_engine_set_sdot)
};

// Row tiles of several CQ matrices that share one input, run as one GEMV
// launch (matrices of one geometry) after at most one activation transform.
// The job table holds `tokens` copies of the pieces, token-major, each over
// its token's input row and into its token's output rows, so a launch over
// the first n tokens runs n times the workgroups of one token.
struct GemvGroup {
    struct Piece {
        const Matrix *m;
        int first, rows;  // rows [first, first + rows) of m
        float *y;         // receives the piece's whole row tiles, from tile first / 256
        int ystride;      // floats between consecutive tokens' outputs
    };
    const Matrix *m0 = nullptr;
    DevBuf<uint8_t> jobs;
    DevBuf<float> rot, big;
    int pieces = 0, per_token = 0;  // jobs and workgroups of one token
    const float *x = nullptr;
    CqJob job0{};
    bool xraw = false;  // groups <= 64: the GEMV transforms the raw input itself

    static bool compatible(const Matrix &a, const Matrix &b) {
        return a.in == b.in && a.bits == b.bits && a.group == b.group &&
               std::memcmp(a.lut, b.lut, sizeof a.lut) == 0;
    }

    // input: [tokens][m.in] rows
    void build(const std::vector<Piece> &ps, const float *input, int tokens) {
        m0 = ps[0].m;
        x = input;
        xraw = gemv_prepass(m0->group) && gemv_quad_takes_x(m0->group, m0->in);
        const bool fused = gemv_fuses_fwht(m0->group) || xraw;
        if (!fused) rot.reserve(size_t(m0->dev) * tokens);
        std::vector<CqJob> host;
        int blocks = 0;
        for (int t = 0; t < tokens; ++t)
            for (const Piece &p : ps) {
                ND_CHECK(compatible(*m0, *p.m), "internal: GEMV group of mixed geometry");
                const int tile0 = p.first / kRowsPerBlock;
                const int tile1 = (p.first + p.rows - 1) / kRowsPerBlock;
                const int tiles = tile1 - tile0 + 1;
                const int rows = std::min(tiles * kRowsPerBlock, p.m->out - tile0 * kRowsPerBlock);
                const float *act = fused ? input + size_t(t) * m0->in : rot.p + size_t(t) * m0->dev;
                host.push_back(CqJob{p.m->codes.p + size_t(tile0) * p.m->chunks * kRowsPerBlock,
                                     p.m->norms.p + size_t(tile0) * p.m->groups * kRowsPerBlock, act,
                                     p.y + size_t(t) * p.ystride, rows, tiles * kRowsPerBlock, blocks, 1});
                blocks += tiles;
            }
        pieces = static_cast<int>(ps.size());
        per_token = blocks / tokens;
        job0 = host[0];
        if (host.size() > 1) {
            jobs.reserve(host.size() * sizeof(CqJob));
            ND_HIP(hipMemcpy(jobs.p, host.data(), host.size() * sizeof(CqJob), hipMemcpyHostToDevice));
        }
    }

    void run(hipStream_t s, int tokens) {
        if (!gemv_fuses_fwht(m0->group) && !xraw) {
            if (gemv_prepass(m0->group))
                launch_rot_many(x, nullptr, tokens, tokens, m0->in, m0->dev, m0->group, m0->scale, rot.p, s);
            else
                m0->transform(x, m0->in, rot.p, tokens, big, s);
        }
        const int njobs = pieces * tokens;
        if (njobs > 1)
            launch_cq_gemv(m0->geom(), CqJob{}, reinterpret_cast<const CqJob *>(jobs.p), njobs, per_token * tokens, s,
                           xraw);
        else
            launch_cq_gemv(m0->geom(), job0, nullptr, 0, per_token, s, xraw);
    }
};

// The int8 ("SDOT") counterpart of GemvGroup (engine.cpp:502-515, 560-577
// with the SDOT path on): the inputs of a launch's tokens transformed and
// quantised by one prepare launch, then the int8 GEMV over the pieces' row
// tiles: one job of batch 1 per piece for a single token (decode step), and
// for a prompt chunk of T tokens one job of batch T per piece
// (engine.cpp:607-640, linear_batch on the SDOT path), so the batch kernels
// decode each code once per batch tile. Both are bit-identical per token.
struct SdotGroup {
    const Matrix *m0 = nullptr;
    SdotGeom g{};
    DevBuf<uint8_t> jobs;
    DevBuf<uint8_t> batched;  // for T = 2 .. tokens: `pieces` jobs of batch T at offset (T - 2) * pieces
    DevBuf<int32_t> q;
    DevBuf<float> xs, xst, rot, big;
    DevBuf<const float *> xptr;
    int pieces = 0, per_token = 0, max_tokens = 0;
    const float *x = nullptr;
    SdotJob job0{};

    void build(const std::vector<GemvGroup::Piece> &ps, const float *input, int tokens) {
        m0 = ps[0].m;
        x = input;
        g = sdot_geom_of(*m0);
        q.reserve(size_t(tokens) * m0->dev / 4);
        xs.reserve(size_t(tokens) * m0->groups);
        rot.reserve(size_t(tokens) * m0->dev);
        std::vector<const float *> rows_in(tokens);
        for (int t = 0; t < tokens; ++t) rows_in[t] = input + size_t(t) * m0->in;
        xptr.reserve(tokens);
        ND_HIP(hipMemcpy(xptr.p, rows_in.data(), tokens * sizeof(const float *), hipMemcpyHostToDevice));
        std::vector<SdotJob> host;
        int blocks = 0;
        for (int t = 0; t < tokens; ++t)
            for (const GemvGroup::Piece &p : ps) {
                ND_CHECK(GemvGroup::compatible(*m0, *p.m), "internal: GEMV group of mixed geometry");
                const int tile0 = p.first / kRowsPerBlock;
                const int tiles = (p.first + p.rows - 1) / kRowsPerBlock - tile0 + 1;
                const int rows = std::min(tiles * kRowsPerBlock, p.m->out - tile0 * kRowsPerBlock);
                const int32_t *qt = q.p + size_t(t) * m0->dev / 4;
                const float *st = xs.p + size_t(t) * m0->groups;  // batch 1: the transposed scales are the same
                host.push_back(SdotJob{p.m->codes.p + size_t(tile0) * p.m->chunks * kRowsPerBlock,
                                       p.m->norms.p + size_t(tile0) * p.m->groups * kRowsPerBlock, qt, st,
                                       p.y + size_t(t) * p.ystride, rows, tiles * kRowsPerBlock, blocks, 1, st, 0,
                                       rows_in[t]});
                blocks += tiles;
            }
        pieces = static_cast<int>(ps.size());
        per_token = blocks / tokens;
        max_tokens = tokens;
        job0 = host[0];
        if (host.size() > 1) {
            jobs.reserve(host.size() * sizeof(SdotJob));
            ND_HIP(hipMemcpy(jobs.p, host.data(), host.size() * sizeof(SdotJob), hipMemcpyHostToDevice));
        }
        // batch jobs: token 0's pieces over all rows of the chunk (q, scales and
        // outputs of consecutive tokens are consecutive rows)
        if (tokens >= 2 && m0->group <= kWindow) {
            xst.reserve(size_t(tokens) * m0->groups);
            std::vector<SdotJob> bt;
            for (int t = 2; t <= tokens; ++t)
                for (int k = 0; k < pieces; ++k) {
                    SdotJob j = host[k];
                    j.batch = t;
                    j.xst = xst.p;
                    j.ystride = ps[k].ystride;
                    bt.push_back(j);
                }
            batched.reserve(bt.size() * sizeof(SdotJob));
            ND_HIP(hipMemcpy(batched.p, bt.data(), bt.size() * sizeof(SdotJob), hipMemcpyHostToDevice));
        }
    }

    // The buffers run() prepares for `tokens` tokens, for a kernel that prepares
    // them itself (groups of 128 or 256 positions).
    bool target(PrepTarget &pt, int tokens) const {
        if ((m0->group != 128 && m0->group != 256) || (tokens >= 2 && !batched.p)) return false;
        pt = PrepTarget{reinterpret_cast<int8_t *>(q.p), xs.p, tokens >= 2 ? xst.p : nullptr, m0->dev, m0->padded,
                        m0->groups, m0->kind, m0->group, m0->scale};
        return true;
    }

    // prepared: the input was prepared into target()'s buffers already
    void run(hipStream_t s, int tokens, bool prepared = false) {
        const bool batch = tokens >= 2 && batched.p;
        if (!prepared && tokens == 1 && sdot_gemv_takes_x(g, per_token, 1)) {  // the GEMV prepares the row itself
            launch_sdot_gemv_x(g, job0, pieces > 1 ? reinterpret_cast<const SdotJob *>(jobs.p) : nullptr,
                               pieces > 1 ? pieces : 0, per_token, s);
            return;
        }
        if (!prepared &&
            !launch_sdot_prepare(nullptr, xptr.p, batch ? tokens : 1, tokens, m0->in, m0->padded, m0->dev, m0->group,
                                 m0->scale, m0->kind, q.p, xs.p, batch ? xst.p : nullptr, s)) {
            ND_CHECK(!batch, "internal: batched int8 prepare refused the group");
            m0->transform(x, m0->in, rot.p, tokens, big, s);
            launch_sdot_quantize(rot.p, m0->dev, tokens, m0->padded, m0->dev, m0->group, m0->kind, q.p, xs.p, s);
        }
        if (batch) {
            const auto *table = reinterpret_cast<const SdotJob *>(batched.p) + size_t(tokens - 2) * pieces;
            launch_sdot_gemv(g, SdotJob{}, table, pieces, per_token, tokens, s);
            return;
        }
        const int njobs = pieces * tokens;
        if (njobs > 1)
            launch_sdot_gemv(g, SdotJob{}, reinterpret_cast<const SdotJob *>(jobs.p), njobs, per_token * tokens, 1, s);
        else
            launch_sdot_gemv(g, job0, nullptr, 0, per_token, 1, s);
    }
};

// GEMVs of several matrices over one input: CQ matrices in as few groups as
// their geometries and paths allow, dense ones through the dense kernel.
struct Projection {
    std::vector<std::unique_ptr<GemvGroup>> groups;
    std::vector<std::unique_ptr<SdotGroup>> groups8;
    struct Dense {
        const float *w;
        int cols, first, rows;
        float *y;
        int ystride;
    };
    std::vector<Dense> dense;
    std::vector<std::vector<GemvGroup::Piece>> pending, pending8;
    const float *x = nullptr;

    // (matrix, first row, rows, output, floats between tokens' outputs)
    void add(const Mat &m, int first, int rows, float *y, int ystride) {
        if (!m.cq) {
            dense.push_back(Dense{m.dense, m.cols, first, rows, y, ystride});
            return;
        }
        auto &pend = m.int8 ? pending8 : pending;
        for (auto &g : pend)
            if (GemvGroup::compatible(*g[0].m, *m.cq)) {
                g.push_back({m.cq, first, rows, y, ystride});
                return;
            }
        pend.push_back({{m.cq, first, rows, y, ystride}});
    }
    void finish(const float *input, int tokens) {
        x = input;
        for (auto &p : pending) {
            groups.push_back(std::make_unique<GemvGroup>());
            groups.back()->build(p, input, tokens);
        }
        for (auto &p : pending8) {
            groups8.push_back(std::make_unique<SdotGroup>());
            groups8.back()->build(p, input, tokens);
        }
        pending.clear();
        pending8.clear();
    }
    // A projection of one int8 group only: the target of the kernel that writes its input.
    bool prep_target(PrepTarget &pt, int tokens) const {
        return groups.empty() && dense.empty() && groups8.size() == 1 && groups8[0]->target(pt, tokens);
    }
    void run(hipStream_t s, int tokens, bool prepared = false) {
        for (auto &g : groups) g->run(s, tokens);
        for (auto &g : groups8) g->run(s, tokens, prepared);
        for (auto &d : dense) launch_eng_dense(d.w, d.cols, d.first, d.rows, x, d.y, d.ystride, tokens, s);
    }
};

}  // namespace

template <class T>
struct BufView {  // a typed range of a buffer owned elsewhere
    T *p = nullptr;
    size_t n = 0;
};

struct GpuEngine {
    EngineConfigC c{};
    int abits = 0, position = 0, prefix = 0, capacity = 0, engring = 1, history_cap = 1;
    int chunk = 1;  // prompt chunk (engine.cpp:1054); the work buffers hold this many tokens
    int ring = 0;   // KV slots past the prefix of a window model: the window plus chunk - 1
    bool int8_kv = false;
    std::vector<int> history;
    std::vector<float> rope_div;
    std::vector<Mat> mats;                 // per tensor (matrix tensors only)
    std::vector<std::unique_ptr<DevBuf<float>>> dense;  // device copies of dense tensors
    std::vector<const float *> dptr;       // per tensor: device fp32 data (dense) or null
    hipStream_t stream = nullptr;
    // The engram work of a launch depends only on the token history: it runs on
    // `side` from the uploaded tokens on, and the main stream waits for site k
    // (ev_site[k]) just before the mixing kernel of layer sites[k].
    hipStream_t side = nullptr;
    hipEvent_t ev_site[kEngMaxSites] = {};
    EngineDims dims{};
    EngineBufs b{};
    DevBuf<float> work;
    DevBuf<int> slots;
    DevBuf<int8_t> kv8;
    DevBuf<float> kv32, kvs;
    std::vector<KvLayer> kv;
    std::vector<LayerDev> layer;
    MhcDev mh{};
    // What a launch reads from the host goes up in one copy: the row ids, then
    // the StepParams, in one pinned buffer and its device twin; the views
    // below point into the two.
    DevBuf<uint8_t> upload, upload_side;  // the step's upload; the side stream's copy of it
    HostBuf<uint8_t> hupload;
    size_t params_offset = 0;  // bytes of upload before the StepParams
    BufView<StepParams> params, hparams;
    BufView<int64_t> ids, hids;  // per chunk: tokens [chunk], then engram rows [sites][chunk][tables]
    DevBuf<float> logits, embed_z, row_scratch, engram_scratch;
    DevBuf<float> attn_scores;  // fp32-KV attention scores past the LDS budget
    HostBuf<float> hlogits, hhidden;
    HostBuf<float> hstep;  // a decode step's logits, written by the LM head kernel itself (pinned)
    std::vector<Projection> mhc_proj, qkvg, oproj;
    std::vector<OutProj> ofused;  // per layer: the out-projection inside the attention launch (codes null: not)
    std::vector<QkvgFused> qfused;  // per layer: its Q|K|V|gate inside the previous post launch (wgs 0: not)
    // the second copy of the state that a fused Q|K|V|gate post writes while its other workgroups read the first
    float *alt_x = nullptr, *alt_u = nullptr, *alt_bx = nullptr, *alt_hpost = nullptr;
    std::vector<std::array<int, 3>> mhc_row;
    const float *phi[3] = {nullptr, nullptr, nullptr};  // dense mHC matrices (null: CQ)
    int mhc_rows[3] = {0, 0, 0};
    std::vector<Projection> engram_kv;
    Projection lm_head;
    Projection lm_head_host;  // the LM head of one token into hstep: no device-to-host copy in a step
    Staging st;  // the engine's own staging (candidate rows)

    int ti(int l) const { return 1 + 14 * l; }
    int mh0() const { return 1 + 14 * c.layers; }
    int engram_base() const { return mh0() + 9; }
    int final_norm() const { return engram_base() + 4 * c.num_sites; }

    GpuEngine(const EngineConfigC &cfg, const TensorDescC *td, int count, int activation_bits);
    ~GpuEngine() {
        if (side) (void)hipStreamSynchronize(side);
        for (hipEvent_t e : ev_site)
            if (e) (void)hipEventDestroy(e);
        if (side) (void)hipStreamDestroy(side);
        if (stream) (void)hipStreamDestroy(stream);
    }
    void reset(int prefix_len);
    // engine.cpp:500 with a ring of `ring` slots: positions inside the window
    // keep distinct slots over a whole chunk
    int cache_slot(int pos) const { return !c.window ? pos : pos < prefix ? pos : prefix + (pos - prefix) % ring; }
    int max_length() const { return c.window ? c.window + prefix : capacity; }
    void set_token(int t, int token);
    void run(int tokens);
    void build_projections();
    OutProj out_projection(const Projection &p) const;
    QkvgFused qkvg_fusion(int l) const;
    void set_sdot();
    void step(int token, float *logits_out, float *hidden_out);
    void prefill(const int *tokens, int num_tokens, bool last_only, float *logits_out, float *hidden_out);
    void project_candidates(const int *candidates, int count, float *out);
    // engine.cpp:410-419: the KV cache plus a cached prefix snapshot
    size_t kv_storage_bytes() const {
        return kv8.n + kv32.n * sizeof(float) + kvs.n * sizeof(float) + snap.k8.n + snap.k32.n * sizeof(float) +
               snap.ks.n * sizeof(float);
    }
    // engine.cpp:450-494: the prefix's KV slots, token history and engram ring
    struct Snapshot {
        bool valid = false, int8 = false;
        int position = 0;
        std::vector<int> history;
        DevBuf<float> k32, ks, ring;  // rows (layer, K | V, kv head) of prefix slots
        DevBuf<int8_t> k8;
    } snap;
    void cache_prefix();
    int reset_to_prefix();
    void import_state(int pos, int pinned, const int *ids, const int *positions, int count, const float *k,
                      const float *v);
    int decode_loop(int first_token, int max_new_tokens, const DfaC *dfa, int *out, int *generated);
    void upload_tokens(int tokens);
    // (on the side stream the kernels read the side stream's own copy of the upload)
    void run_engram_site(int site, int tokens, hipStream_t s, bool side_copy = false);
    // copies `prefix` slots of every (layer, K | V, kv head) row between the cache and the snapshot
    void copy_prefix_slots(bool to_snapshot);
};

GpuEngine::GpuEngine(const EngineConfigC &cfg, const TensorDescC *td, int count, int activation_bits)
    : c(cfg), abits(activation_bits) {
    ND_CHECK(td && count > 0, "engine: no tensors");
    ND_CHECK(abits == 0 || abits == 8, "engine: activation bits must be 0 or 8");
    const int D = c.dim, N = c.lanes, HD = c.head_dim, A = c.heads * HD, K = c.kvheads * HD;
    ND_CHECK(D > 0 && (N == 1 || N == 2 || N == 4 || N == 8) && c.layers > 0 && c.heads > 0 && c.kvheads > 0 &&
                 c.heads % c.kvheads == 0 && c.heads / c.kvheads <= 8,
             "engine: unsupported geometry (mHC lanes 1, 2, 4 or 8; at most 8 heads per kv head)");
    ND_CHECK(HD % 4 == 0 && HD <= 2 * kEngMaxHalfHd && D <= kEngThreads && c.hada >= D && c.hada <= 4096 &&
                 (c.hada & (c.hada - 1)) == 0,
             "engine: unsupported head / Hadamard geometry");
    ND_CHECK(c.num_sites >= 0 && c.num_sites <= kEngMaxSites && c.num_orders >= 0 && c.num_orders <= 4,
             "engine: unsupported engram geometry");
    ND_CHECK(!c.num_sites || (c.tables > 0 && c.tables <= kEngMaxTables && c.num_orders > 0 &&
                              c.tables % c.num_orders == 0 && c.tables * c.subdim == D && c.taps > 0 &&
                              c.taps <= kEngMaxTaps && c.dilation > 0),
             "engine: unsupported engram geometry");
    for (int k = 0; k < c.num_sites; ++k) {
        ND_CHECK(c.sites[k] >= 0 && c.sites[k] < c.layers, "engine: engram site outside the layers");
        for (int j = 0; j < k; ++j)
            ND_CHECK(c.sites[j] != c.sites[k], "engine: two engram sites on one layer (the archive format forbids it)");
    }
    ND_CHECK(count >= final_norm() + 1, "engine: tensor count does not match the geometry");
    ND_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    if (c.num_sites) {
        ND_HIP(hipStreamCreateWithFlags(&side, hipStreamNonBlocking));
        for (int k = 0; k < c.num_sites; ++k) ND_HIP(hipEventCreateWithFlags(&ev_site[k], hipEventDisableTiming));
    }

    // tensors: matrices keep the caller's CQ handle; dense data goes to the device as fp32
    mats.resize(count);
    dense.resize(count);
    dptr.assign(count, nullptr);
    for (int i = 0; i < count; ++i) {
        mats[i].rows = td[i].rows;
        mats[i].cols = td[i].cols;
        if (td[i].cq) {
            mats[i].cq = &static_cast<CqHandle *>(td[i].cq)->m;
        } else {
            ND_CHECK(td[i].data, "engine: tensor without data");
            dense[i] = std::make_unique<DevBuf<float>>();
            dense[i]->reserve(size_t(td[i].rows) * td[i].cols);
            ND_HIP(hipMemcpy(dense[i]->p, td[i].data, size_t(td[i].rows) * td[i].cols * sizeof(float),
                             hipMemcpyHostToDevice));
            dptr[i] = dense[i]->p;
            mats[i].dense = dense[i]->p;
        }
    }
    auto vec = [&](int i) {
        ND_CHECK(dptr[i], "engine: vector tensors must be dense");
        return dptr[i];
    };
    auto mat = [&](int i, int rows, int cols) -> const Mat & {
        const Mat &m = mats[i];
        if (m.cq) {
            ND_CHECK(m.cq->out == rows && m.cq->in == cols, "engine: CQ matrix shape does not match the geometry");
        } else {
            ND_CHECK(m.rows * m.cols == rows * cols, "engine: dense matrix shape does not match the geometry");
        }
        return m;
    };

    dims.D = D;
    dims.N = N;
    dims.H = c.heads;
    dims.KV = c.kvheads;
    dims.HD = HD;
    dims.A = A;
    dims.K = K;
    dims.hada = c.hada;
    dims.layers = c.layers;
    dims.tables = c.tables;
    dims.subdim = c.subdim;
    dims.taps = c.taps;
    dims.abits = abits;
    dims.sqrt_d = std::sqrt(float(D));
    dims.inv_hada = 1 / std::sqrt(float(c.hada));
    dims.scale = 1 / std::sqrt(float(HD));
    dims.ogroups = 0;
    engring = int(int64_t(c.taps - 1) * c.dilation + 1);
    ND_CHECK(engring >= 1, "invalid Engram ring size");
    dims.engring = engring;
    int max_order = 1;
    for (int i = 0; i < c.num_orders; ++i) max_order = std::max(max_order, c.orders[i]);
    history_cap = c.num_sites ? engring + max_order - 1 : 1;
    history.assign(history_cap, 0);
    rope_div.resize(HD / 2);
    for (int j = 0; j < HD / 2; ++j) rope_div[j] = std::pow(c.rope_theta, float(2 * j) / HD);  // engine.cpp:400

    // work buffers (one allocation), `chunk` tokens each
    chunk = c.window ? std::min(kEngMaxChunk, c.window) : kEngMaxChunk;
    {  // the score buffer of the longest slot list a reset can make (a prefix of up to max_seq)
        const size_t G = size_t(c.heads / c.kvheads);
        const size_t longest = size_t(c.window ? c.window + c.max_seq : c.max_seq);
        if (G * longest * sizeof(float) > kEngScoreLds) {
            const size_t per_token = size_t(c.kvheads) * G * longest * sizeof(float);
            chunk = int(std::min<size_t>(chunk, std::max<size_t>(kEngMinChunk, kEngScoreBudget / per_token)));
        }
    }
    const int mhc_tiles = 2 * kRowsPerBlock;  // a piece spans at most two row tiles
    const int sites = std::max(1, c.num_sites);
    dims.sites = sites;
    dims.mhc_stride = mhc_tiles;
    size_t off = 0;
    auto take = [&](size_t n) {
        const size_t at = off;
        off += (n * chunk + 63) / 64 * 64;
        return at;
    };
    const size_t ox = take(N * D), onx = take(N * D), ou = take(D), obx = take(D), oz = take(D), oq = take(A),
                 ok = take(K), ov = take(K), og = take(A), oa = take(A), op = take(D), oh = take(size_t(c.layers) * D),
                 ohp = take(N), ohq = take(N), ohr = take(N * N), oht = take(N * N), om0 = take(mhc_tiles),
                 om1 = take(mhc_tiles),
                 om2 = take(mhc_tiles), oe = take(D), oek = take(size_t(sites) * D), oev = take(size_t(sites) * D),
                 orv = take(D), ozf = take(D), oop = take(size_t(c.kvheads) * D), ox2 = take(N * D), ou2 = take(D),
                 obx2 = take(D), ohq2 = take(N);
    const size_t oring = off;  // shared by the chunk
    off += (size_t(sites) * engring * D + 63) / 64 * 64;
    work.reserve(off);
    ND_HIP(hipMemset(work.p, 0, off * sizeof(float)));
    float *w = work.p;
    b.x = w + ox;
    b.oparts = w + oop;
    alt_x = w + ox2;
    alt_u = w + ou2;
    alt_bx = w + obx2;
    alt_hpost = w + ohq2;
    b.nx = w + onx;
    b.u = w + ou;
    b.bx = w + obx;
    b.z = w + oz;
    b.q = w + oq;
    b.k = w + ok;
    b.v = w + ov;
    b.gate = w + og;
    b.att = w + oa;
    b.proj = w + op;
    b.hidden = w + oh;
    b.hpre = w + ohp;
    b.hpost = w + ohq;
    b.hres = w + ohr;
    b.hroute = w + oht;
    b.mhc_out[0] = w + om0;
    b.mhc_out[1] = w + om1;
    b.mhc_out[2] = w + om2;
    b.e = w + oe;
    b.ek = w + oek;
    b.ev = w + oev;
    b.rawv = w + orv;
    b.engring = w + oring;
    b.zf = w + ozf;
    {
        const size_t nids = size_t(chunk) * (1 + size_t(sites) * std::max(1, c.tables));
        params_offset = (nids * sizeof(int64_t) + 255) & ~size_t(255);
        const size_t bytes = params_offset + size_t(chunk) * sizeof(StepParams);
        upload.reserve(bytes);
        upload_side.reserve(bytes);
        hupload.reserve(bytes);
        std::memset(hupload.p, 0, bytes);
        ids = {reinterpret_cast<int64_t *>(upload.p), nids};
        hids = {reinterpret_cast<int64_t *>(hupload.p), nids};
        params = {reinterpret_cast<StepParams *>(upload.p + params_offset), size_t(chunk)};
        hparams = {reinterpret_cast<StepParams *>(hupload.p + params_offset), size_t(chunk)};
    }
    logits.reserve(size_t(chunk) * c.vocab);
    embed_z.reserve(size_t(chunk) * D);

    // layers
    const int mhi = mh0();
    mh.a_pre = vec(mhi);
    mh.a_post = vec(mhi + 1);
    mh.a_res = vec(mhi + 2);
    mh.b_pre = vec(mhi + 3);
    mh.b_post = vec(mhi + 4);
    mh.b_res = vec(mhi + 5);
    layer.resize(c.layers);
    mhc_proj.resize(c.layers);
    qkvg.resize(c.layers);
    oproj.resize(c.layers);
    mhc_row.resize(c.layers);
    for (int l = 0; l < c.layers; ++l) {
        const int t0 = ti(l);
        LayerDev &L = layer[l];
        L.norm_in = vec(t0);
        L.q_norm = vec(t0 + 4);
        L.k_norm = vec(t0 + 5);
        L.post_norm = vec(t0 + 8);
        L.attn_gate = vec(t0 + 9);
        L.pre_hada = vec(t0 + 10);
        L.d1 = vec(t0 + 11);
        L.d2 = vec(t0 + 12);
        L.d3 = vec(t0 + 13);
        (void)mat(t0 + 1, A, D), (void)mat(t0 + 2, K, D), (void)mat(t0 + 3, K, D), (void)mat(t0 + 6, A, D);
        (void)mat(t0 + 7, D, A);
        const int rows[3] = {N, N, N * N};
        for (int m = 0; m < 3; ++m) {
            const Mat &M = mat(mhi + 6 + m, c.layers * rows[m], N * D);
            const int first = l * rows[m];
            // the GEMV's row tiles; dense rows go through one multi-matrix launch
            mhc_row[l][m] = M.cq ? first - first / kRowsPerBlock * kRowsPerBlock : 0;
            phi[m] = M.cq ? nullptr : M.dense;
            mhc_rows[m] = rows[m];
        }
    }
    for (int s = 0; s < c.num_sites; ++s) {
        ND_CHECK(c.sites[s] >= 0 && c.sites[s] < c.layers, "engine: engram site outside the layers");
        const int e0 = engram_base() + 4 * s;
        ND_CHECK(mats[e0].cq ? mats[e0].cq->in == c.subdim : mats[e0].cols == c.subdim,
                 "engine: engram tables shape does not match the geometry");
        (void)vec(e0 + 3);
        (void)mat(e0 + 1, D, D), (void)mat(e0 + 2, D, D);
        if (mats[e0].cq) engram_scratch.reserve(size_t(chunk) * c.tables * mats[e0].cq->padded);
    }
    (void)vec(final_norm());
    (void)mat(0, c.vocab, D);
    if (mats[0].cq) row_scratch.reserve(std::max(row_scratch.n, size_t(chunk) * mats[0].cq->padded));
    build_projections();
    reset(0);
}

// The GEMV launches of every projection over the chunk's buffers, each CQ
// matrix on its path (FP32 or int8).
void GpuEngine::build_projections() {
    const int D = c.dim, N = c.lanes, A = c.heads * c.head_dim, K = c.kvheads * c.head_dim;
    const int mhi = mh0();
    for (auto *v : {&mhc_proj, &qkvg, &oproj, &engram_kv}) v->clear();
    ofused.clear();
    qfused.clear();
    mhc_proj.resize(c.layers);
    qkvg.resize(c.layers);
    oproj.resize(c.layers);
    engram_kv.resize(c.num_sites);
    lm_head = Projection{};
    for (int l = 0; l < c.layers; ++l) {
        const int t0 = ti(l);
        qkvg[l].add(mats[t0 + 1], 0, A, b.q, A);
        qkvg[l].add(mats[t0 + 2], 0, K, b.k, K);
        qkvg[l].add(mats[t0 + 3], 0, K, b.v, K);
        qkvg[l].add(mats[t0 + 6], 0, A, b.gate, A);
        qkvg[l].finish(b.z, chunk);
        oproj[l].add(mats[t0 + 7], 0, D, b.proj, D);
        oproj[l].finish(b.att, chunk);
        ofused.push_back(out_projection(oproj[l]));
        qfused.push_back(qkvg_fusion(l));
        const int rows[3] = {N, N, N * N};
        for (int m = 0; m < 3; ++m)
            if (mats[mhi + 6 + m].cq) mhc_proj[l].add(mats[mhi + 6 + m], l * rows[m], rows[m], b.mhc_out[m], dims.mhc_stride);
        mhc_proj[l].finish(b.nx, chunk);
    }
    for (int s = 0; s < c.num_sites; ++s) {
        const int e0 = engram_base() + 4 * s;
        engram_kv[s].add(mats[e0 + 1], 0, D, b.ek + s * D, dims.sites * D);
        engram_kv[s].add(mats[e0 + 2], 0, D, b.rawv, D);
        engram_kv[s].finish(b.e, chunk);
    }
    lm_head.add(mats[0], 0, c.vocab, logits.p, c.vocab);
    lm_head.finish(b.zf, chunk);
    hstep.reserve(c.vocab);  // allocated once: the job tables below hold its address
    lm_head_host = Projection{};
    lm_head_host.add(mats[0], 0, c.vocab, hstep.p, c.vocab);
    lm_head_host.finish(b.zf, 1);
}

// The out-projection runs inside the attention launch (OutProj) when it is one
// FP32 CQ matrix of 2- or 4-bit codes whose groups of 128 positions are the
// G query heads of one kv head, with at most 512 rows and no activation
// quantiser before it (NEEDLE2_ENGINE_OPROJ=gemv: always the separate GEMV).
OutProj GpuEngine::out_projection(const Projection &p) const {
    OutProj op{};
    const char *mode = std::getenv("NEEDLE2_ENGINE_OPROJ");
    if (mode && std::strcmp(mode, "gemv") == 0) return op;
    if (p.groups.size() != 1 || !p.groups8.empty() || !p.dense.empty() || p.groups[0]->pieces != 1) return op;
    const Matrix &m = *p.groups[0]->m0;
    const int G = c.heads / c.kvheads;
    if (abits || G * c.head_dim != 128 || m.group != 128 || m.in != c.heads * c.head_dim || m.out != c.dim ||
        m.out > 512 || c.kvheads > 8 || (m.kind != kNib && m.kind != kCrumb))
        return op;
    const CqGeom g = m.geom();
    op.codes = m.codes.p;
    op.norms = m.norms.p;
    op.parts = b.oparts;
    op.rows = m.out;
    op.chunks = g.chunks;
    op.groups = g.groups;
    op.kind = g.kind;
    op.scale = g.scale;
    for (int i = 0; i < 16; ++i) op.lut[i] = g.lut[i];
    // a decode step's rows over 2^split workgroups per kv head (NEEDLE2_ENGINE_OSPLIT: 0, 1 or 2)
    const char *split = std::getenv("NEEDLE2_ENGINE_OSPLIT");
    op.split_shift = split ? std::min(2, std::max(0, std::atoi(split))) : 1;
    return op;
}

// Layer l's Q|K|V|gate runs inside the previous layer's post launch (layer
// 0's: inside the launch that starts the lanes and mixes; QkvgFused) when its
// four matrices are one FP32 GEMV group of 2- or 4-bit codes in groups of 128
// over d_model <= 512 (a multiple of 128) inputs, with no activation
// quantiser (NEEDLE2_ENGINE_QKVG=gemv: always the separate GEMV); the step
// takes it where the post / mixing launch is fused.
QkvgFused GpuEngine::qkvg_fusion(int l) const {
    QkvgFused q{};
    const char *mode = std::getenv("NEEDLE2_ENGINE_QKVG");
    if (mode && std::strcmp(mode, "gemv") == 0) return q;
    const Projection &p = qkvg[l];
    if (abits || p.groups.size() != 1 || !p.groups8.empty() || !p.dense.empty() ||
        p.groups[0]->pieces != 4 || c.dim > 512 || c.dim % 128)
        return q;
    const int t0 = ti(l), idx[4] = {t0 + 1, t0 + 2, t0 + 3, t0 + 6};
    float *ys[4] = {b.q, b.k, b.v, b.gate};
    const Matrix &m0 = *mats[idx[0]].cq;
    if (m0.group != 128 || m0.in != c.dim || (m0.kind != kNib && m0.kind != kCrumb)) return q;
    const CqGeom g = m0.geom();
    int wgs = 0;
    for (int k = 0; k < 4; ++k) {
        const Matrix *m = mats[idx[k]].cq;
        if (!m || !GemvGroup::compatible(m0, *m)) return QkvgFused{};
        q.piece[k] = QkvgPiece{reinterpret_cast<const uint4 *>(m->codes.p), m->norms.p, ys[k], m->out, wgs};
        wgs += (m->out + kQkvgRows - 1) / kQkvgRows;
    }
    q.pieces = 4;
    q.wgs = wgs;
    q.chunks = g.chunks;
    q.groups = g.groups;
    q.kind = g.kind;
    q.scale = g.scale;
    for (int i = 0; i < 16; ++i) q.lut[i] = g.lut[i];
    return q;
}

// engine.cpp:424-432: the int8 path for the CQ matrices of 2- or 4-bit codes
// and groups of 64 .. 131072 (the rest stay FP32), for every later step.
void GpuEngine::set_sdot() {
    for (Mat &m : mats)
        if (m.cq && (m.cq->bits == 2 || m.cq->bits == 4) && m.cq->group >= 64 && m.cq->group <= 131072) m.int8 = true;
    ND_HIP(hipStreamSynchronize(stream));
    build_projections();
}

void GpuEngine::reset(int prefix_len) {
    ND_CHECK(prefix_len >= 0 && prefix_len <= c.max_seq, "prefix length outside [0, max_seq]");
    snap.valid = false;
    snap.k32.release();
    snap.k8.release();
    snap.ks.release();
    snap.ring.release();
    position = 0;
    prefix = prefix_len;
    std::fill(history.begin(), history.end(), 0);
    // engine.cpp:433-449, with chunk - 1 more ring slots for a window model
    ring = c.window ? c.window + chunk - 1 : 0;
    capacity = c.window ? ring + prefix : c.max_seq;
    dims.capacity = capacity;
    const int G = c.heads / c.kvheads;
    // attention scores past the LDS budget go to a device buffer (any context)
    if (size_t(G) * max_length() * sizeof(float) > kEngScoreLds)
        attn_scores.reserve(size_t(chunk) * c.kvheads * G * max_length());
    else
        attn_scores.release();
    const size_t per_layer = size_t(c.kvheads) * capacity * c.head_dim;
    const size_t scales = size_t(c.kvheads) * capacity;
    kv.assign(c.layers, KvLayer{});
    if (int8_kv) {
        kv32.release();
        kv8.reserve(2 * per_layer * c.layers);
        kvs.reserve(2 * scales * c.layers);
        for (int l = 0; l < c.layers; ++l) {
            kv[l].k8 = kv8.p + 2 * per_layer * l;
            kv[l].v8 = kv[l].k8 + per_layer;
            kv[l].ks = kvs.p + 2 * scales * l;
            kv[l].vs = kv[l].ks + scales;
        }
    } else {
        kv8.release();
        kvs.release();
        kv32.reserve(2 * per_layer * c.layers);
        for (int l = 0; l < c.layers; ++l) {
            kv[l].k32 = kv32.p + 2 * per_layer * l;
            kv[l].v32 = kv[l].k32 + per_layer;
        }
    }
    slots.reserve(size_t(chunk) * capacity);
    b.slots = slots.p;
    if (c.num_sites) ND_HIP(hipMemsetAsync(b.engring, 0, size_t(c.num_sites) * engring * c.dim * sizeof(float), stream));
    ND_HIP(hipStreamSynchronize(stream));
}

void GpuEngine::copy_prefix_slots(bool to_snapshot) {
    const size_t rows = size_t(c.layers) * 2 * c.kvheads, HD = c.head_dim, P = prefix;
    auto copy = [&](void *cache, void *saved, size_t elem, size_t per_slot) {
        const size_t cache_pitch = size_t(capacity) * per_slot * elem, saved_pitch = P * per_slot * elem;
        if (to_snapshot)
            ND_HIP(hipMemcpy2DAsync(saved, saved_pitch, cache, cache_pitch, saved_pitch, rows, hipMemcpyDeviceToDevice,
                                    stream));
        else
            ND_HIP(hipMemcpy2DAsync(cache, cache_pitch, saved, saved_pitch, saved_pitch, rows, hipMemcpyDeviceToDevice,
                                    stream));
    };
    if (int8_kv) {
        copy(kv8.p, snap.k8.p, 1, HD);
        copy(kvs.p, snap.ks.p, sizeof(float), 1);
    } else {
        copy(kv32.p, snap.k32.p, sizeof(float), HD);
    }
    const size_t ring_floats = size_t(c.num_sites) * engring * c.dim;
    if (ring_floats) {
        if (to_snapshot)
            ND_HIP(hipMemcpyAsync(snap.ring.p, b.engring, ring_floats * sizeof(float), hipMemcpyDeviceToDevice, stream));
        else
            ND_HIP(hipMemcpyAsync(b.engring, snap.ring.p, ring_floats * sizeof(float), hipMemcpyDeviceToDevice, stream));
    }
    ND_HIP(hipStreamSynchronize(stream));
}

void GpuEngine::cache_prefix() {
    if (position <= 0 || position != prefix) throw Error("prefix snapshot requires position == prefix_len > 0");
    const size_t rows = size_t(c.layers) * 2 * c.kvheads;
    snap.valid = false;
    if (int8_kv) {
        snap.k32.release();
        snap.k8.reserve(rows * prefix * c.head_dim);
        snap.ks.reserve(rows * prefix);
    } else {
        snap.k8.release();
        snap.ks.release();
        snap.k32.reserve(rows * prefix * c.head_dim);
    }
    snap.ring.reserve(std::max<size_t>(1, size_t(c.num_sites) * engring * c.dim));
    copy_prefix_slots(true);
    snap.history = history;
    snap.position = position;
    snap.int8 = int8_kv;
    snap.valid = true;
}

int GpuEngine::reset_to_prefix() {
    if (!snap.valid) throw Error("no cached prefix; call cache_prefix() after consuming the complete prefix");
    const int cached = snap.position;
    if (prefix != cached || snap.int8 != int8_kv || capacity != (c.window ? ring + cached : c.max_seq))
        throw Error("cached prefix geometry no longer matches the current state");
    copy_prefix_slots(false);
    history = snap.history;
    position = cached;
    return position;
}

// engine.cpp:784-815: a state computed elsewhere (the torch prefill): position
// `pos` after `pinned` prefix tokens, the token history from ids, fp32 K / V
// rows [layers][count][kv heads * head_dim] for the cache slots of
// positions[count] (stored as the step stores them, fp32 or int8), and the
// engram ring recomputed for the last ring positions.
void GpuEngine::import_state(int pos, int pinned, const int *ids, const int *positions, int count, const float *k,
                             const float *v) {
    ND_CHECK(pos >= 0 && count >= 0 && (!pos || ids) && (!count || (positions && k && v)), "import: invalid state");
    reset(pinned);
    for (int i = 0; i < pos; ++i) ND_CHECK(ids[i] >= 0 && ids[i] < c.vocab, "token outside vocabulary");
    const int K = c.kvheads * c.head_dim;
    for (int t = 0; t < count; ++t) ND_CHECK(positions[t] >= 0 && cache_slot(positions[t]) < capacity,
                                             "import: position outside the cache");
    for (int i = std::max(0, pos - history_cap); i < pos; ++i) history[i % history_cap] = ids[i];
    if (count > 0) {
        const size_t n = size_t(c.layers) * count * K;
        DevBuf<float> dk, dv;
        DevBuf<int> dslots;
        dk.reserve(n);
        dv.reserve(n);
        dslots.reserve(count);
        std::vector<int> hs(count);
        for (int t = 0; t < count; ++t) hs[t] = cache_slot(positions[t]);
        ND_HIP(hipMemcpyAsync(dk.p, k, n * sizeof(float), hipMemcpyHostToDevice, stream));
        ND_HIP(hipMemcpyAsync(dv.p, v, n * sizeof(float), hipMemcpyHostToDevice, stream));
        ND_HIP(hipMemcpyAsync(dslots.p, hs.data(), count * sizeof(int), hipMemcpyHostToDevice, stream));
        for (int l = 0; l < c.layers; ++l)
            launch_eng_kv_import(dk.p + size_t(l) * count * K, dv.p + size_t(l) * count * K, dslots.p, count, kv[l],
                                 dims, stream);
        ND_HIP(hipStreamSynchronize(stream));
    }
    // only raw engram values persist: recompute the ring rows of the last positions
    const int first = std::max(0, pos - engring);
    if (c.num_sites && first < pos) {
        for (int p0 = first; p0 < pos; p0 += chunk) {
            const int T = std::min(chunk, pos - p0);
            position = p0;
            for (int t = 0; t < T; ++t) set_token(t, ids[p0 + t]);
            upload_tokens(T);
            for (int site = 0; site < c.num_sites; ++site) run_engram_site(site, T, stream);
            ND_HIP(hipStreamSynchronize(stream));  // the host rewrites the token buffers next chunk
        }
    }
    position = pos;
}

// engine.cpp:1360-1497: greedy decoding from first_token until eos / stop,
// max_new_tokens (the first token included) or a terminal grammar state; a
// grammar state with exact candidates projects only those rows.
int GpuEngine::decode_loop(int first_token, int max_new_tokens, const DfaC *dfa, int *out, int *generated) {
    if (max_new_tokens <= 0) {
        if (generated) *generated = 0;
        return 0;
    }
    if (first_token < 0 || first_token >= c.vocab) throw Error("token outside vocabulary");
    auto check_tokens = [&](const int *ids, int n) {
        for (int i = 0; i < n; ++i)
            if (ids[i] < 0 || ids[i] >= c.vocab) throw Error("candidate outside vocabulary");
    };
    if (dfa) {
        if (dfa->num_states <= 0 || dfa->initial_state < 0 || dfa->initial_state >= dfa->num_states ||
            !dfa->state_types || !dfa->fallback_next_states || !dfa->candidate_offsets)
            throw Error("invalid DFA states");
        for (int token : {dfa->eos_id, dfa->stop_id, dfa->tool_start_id, dfa->tool_end_id})
            if (token < 0 || token >= c.vocab) throw Error("DFA token outside vocabulary");
        if (dfa->candidate_offsets[0] != 0) throw Error("invalid DFA offsets");
        for (int st8 = 0; st8 < dfa->num_states; ++st8) {
            const int type = dfa->state_types[st8], fallback = dfa->fallback_next_states[st8];
            const int begin = dfa->candidate_offsets[st8], end = dfa->candidate_offsets[st8 + 1];
            if ((type != 0 && type != 1 && type != 4) || fallback < -1 || fallback >= dfa->num_states || begin < 0 ||
                end < begin)
                throw Error("invalid DFA state");
            if (type == 1 && begin == end) throw Error("DFA state has no candidates");
            if (end > begin) {
                if (!dfa->candidate_tokens || !dfa->next_states) throw Error("missing DFA transitions");
                check_tokens(dfa->candidate_tokens + begin, end - begin);
            }
            for (int i = begin; i < end; ++i)
                if (dfa->next_states[i] < 0 || dfa->next_states[i] >= dfa->num_states)
                    throw Error("invalid DFA transition");
        }
    }
    const int eos = dfa ? dfa->eos_id : 1, stop = dfa ? dfa->stop_id : 5;
    // the transition of `state` on `token`, or -1 when the state lists no such candidate
    auto transition = [&](int state, int token) {
        for (int i = dfa->candidate_offsets[state]; i < dfa->candidate_offsets[state + 1]; ++i)
            if (dfa->candidate_tokens[i] == token) return dfa->next_states[i];
        return -1;
    };
    auto argmax = [](const float *x, int n) {
        int best = 0;
        for (int i = 1; i < n; ++i)
            if (x[i] > x[best]) best = i;
        return best;
    };
    int count = 0;
    out[count++] = first_token;
    if (first_token == eos || first_token == stop) {
        if (generated) *generated = count;
        return 0;
    }
    int state = 0;
    if (dfa) {
        state = dfa->initial_state;
        const int next = transition(state, first_token);
        if (next >= 0) {
            state = next;
        } else {
            if (dfa->state_types[state] != 0) throw Error("first token rejected by DFA");
            if (dfa->fallback_next_states[state] >= 0) state = dfa->fallback_next_states[state];
        }
    }
    // a state may list more candidates than the vocabulary (duplicates are valid): the score buffer
    // holds the full logits or the largest candidate list, whichever is longer
    size_t score_len = size_t(c.vocab);
    if (dfa)
        for (int st8 = 0; st8 < dfa->num_states; ++st8)
            score_len = std::max(score_len, size_t(dfa->candidate_offsets[st8 + 1] - dfa->candidate_offsets[st8]));
    std::vector<float> scores(score_len);
    int token = first_token;
    while (count < max_new_tokens) {
        const int type = dfa ? dfa->state_types[state] : 0;
        if (type == 4) break;
        int next_token;
        if (type == 0) {
            step(token, scores.data(), nullptr);
            next_token = argmax(scores.data(), c.vocab);
            if (dfa) {
                const int next = transition(state, next_token);
                if (next >= 0) state = next;
                else if (dfa->fallback_next_states[state] >= 0) state = dfa->fallback_next_states[state];
            }
        } else {
            const int begin = dfa->candidate_offsets[state], n = dfa->candidate_offsets[state + 1] - begin;
            const int *cands = dfa->candidate_tokens + begin;
            int pick = 0;
            if (n == 1) {
                step(token, nullptr, nullptr);
            } else {
                step(token, nullptr, nullptr);
                project_candidates(cands, n, scores.data());
                pick = argmax(scores.data(), n);
            }
            next_token = cands[pick];
            state = dfa->next_states[begin + pick];
        }
        out[count++] = next_token;
        token = next_token;
        if (next_token == eos || next_token == stop || (dfa && dfa->state_types[state] == 4)) break;
    }
    if (generated) *generated = count;
    return 0;
}

// Token t of the next launch: its StepParams and row ids (engine.cpp:
// 755-781, 898-911, 968-975; the token history advances here, in order).
void GpuEngine::set_token(int t, int token) {
    const int HD = c.head_dim, pos = position + t;
    history[pos % history_cap] = token;
    StepParams &p = hparams.p[t];
    hids.p[t] = token;
    p.position = pos;
    p.slot = cache_slot(pos);
    p.prefix = prefix;
    p.window = c.window;
    p.ring = ring;
    p.chunk_start = position;
    p.prefix_count = c.window ? std::min(prefix, pos + 1) : 0;  // engine.cpp:900-902
    p.start = c.window ? std::max(prefix, pos - c.window + 1) : 0;
    p.length = p.prefix_count + std::max(0, pos - p.start + 1);
    for (int j = 0; j < HD / 2; ++j) {
        const float a = pos / rope_div[j];
        p.rope_cos[j] = std::cos(a);
        p.rope_sin[j] = std::sin(a);
    }
    if (c.num_sites) {  // engine.cpp:755-781
        const int heads = c.tables / c.num_orders;
        auto hist = [&](int q) { return history[((q % history_cap) + history_cap) % history_cap]; };
        for (int s = 0; s < c.num_sites; ++s) {
            int64_t *rows = hids.p + chunk + (size_t(s) * chunk + t) * c.tables;
            p.engram_zero[s] = 0;
            for (int table = 0; table < c.tables; ++table) {
                const int order = c.orders[table / heads];
                rows[table] = 0;
                if (pos + 1 < order || (c.window && order - 1 >= c.window && pos - order + 1 >= prefix)) {
                    p.engram_zero[s] |= 1 << table;
                    continue;
                }
                uint32_t acc = uint32_t(0x9e3779b9) * uint32_t(table + 1);
                for (int j = 0; j < order; ++j) acc = (acc ^ uint32_t(hist(pos - j))) * uint32_t(0x01000193);
                acc ^= acc >> 15;
                rows[table] = int64_t(table) * c.slots + acc % uint32_t(c.slots);
            }
        }
        for (int tap = 0; tap < c.taps; ++tap) {
            const int past = pos - tap * c.dilation;
            const bool live = past >= 0 && (!c.window || tap * c.dilation < c.window || past < prefix);
            p.tap_pos[tap] = live ? past : -1;
        }
    }
}

// The StepParams and row ids of the first T tokens, to the device.
void GpuEngine::upload_tokens(int T) {
    ND_HIP(hipMemcpyAsync(upload.p, hupload.p, params_offset + size_t(T) * sizeof(StepParams), hipMemcpyHostToDevice,
                          stream));
}

// Engram rows, their quantiser, key / value projections, the conv and the ring
// of one site for the T uploaded tokens (engine.cpp:755-781).
void GpuEngine::run_engram_site(int site, int T, hipStream_t s, bool side_copy) {
    const uint8_t *base = side_copy ? upload_side.p : upload.p;
    const StepParams *dp = reinterpret_cast<const StepParams *>(base + params_offset);
    {
        const int e0 = engram_base() + 4 * site;
        const Mat &tab = mats[e0];
        const int64_t *rows = reinterpret_cast<const int64_t *>(base) + chunk + size_t(site) * chunk * c.tables;
        if (tab.cq)
            launch_cq_rows(tab.cq->geom(), tab.cq->codes.p, tab.cq->norms.p, rows, T * c.tables, c.subdim,
                           tab.cq->padded, engram_scratch.p, b.e, s);
        else
            launch_eng_dense_rows(tab.dense, c.subdim, rows, T * c.tables, b.e, s);
        launch_eng_engram_in(b, dp, site, dims, T, s);
        engram_kv[site].run(s, T);
        launch_eng_engram_out(b, dptr[e0 + 3], dp, site, dims, T, s);
    }
}

// The layers for the `tokens` tokens set by set_token (engine.cpp:968-1040 for
// one token, 1056-1258 for a chunk), leaving each token's final normed hidden
// state in zf. Tokens share nothing but the KV cache and the engram ring, which
// every token of the chunk writes before any reads them.
void GpuEngine::run(int tokens) {
    const int D = c.dim, HD = c.head_dim, T = tokens;
    hipStream_t s = stream;
    upload_tokens(T);
    const StepParams *dp = params.p;

    // a layer's post runs with the next layer's mHC projections and mixing (and the first layer's with
    // the lanes' start) when those are dense and the geometry fits the fused kernel
    const bool fuse = phi[0] && phi[1] && phi[2] && eng_post_mix_fits(dims);
    // embedding rows, lanes (engine.cpp:972-974); a CQ embedding of d_model <= 512 (no padding) is decoded
    // inside the first layer's launch
    const Mat &emb = mats[0];
    EmbedRows er{};
    if (fuse && emb.cq && D <= 512 && emb.cq->padded == D && emb.cq->group <= D)
        er = EmbedRows{emb.cq->codes.p, emb.cq->norms.p, ids.p, embed_z.p, emb.cq->geom()};
    else if (emb.cq)
        launch_cq_rows(emb.cq->geom(), emb.cq->codes.p, emb.cq->norms.p, ids.p, T, D, emb.cq->padded,
                       row_scratch.p, embed_z.p, s);
    else
        launch_eng_dense_rows(emb.dense, D, ids.p, T, embed_z.p, s);
    if (!fuse) launch_eng_start(embed_z.p, b, dims, T, s);
    // engram sites up to layer `upto` onto the side stream, behind its own copy of the upload (a wait
    // for the main stream's copy cost the host ~14 us to issue, which held back the next layer's launches
    // while the GPU idled); the first site issues the copy
    bool sent[kEngMaxSites] = {}, side_copied = false;
    auto send_sites = [&](int upto) {
        for (int k = 0; k < c.num_sites; ++k)
            if (!sent[k] && c.sites[k] <= upto) {
                if (!side_copied) {
                    ND_HIP(hipMemcpyAsync(upload_side.p, hupload.p, params_offset + size_t(T) * sizeof(StepParams),
                                          hipMemcpyHostToDevice, side));
                    side_copied = true;
                }
                run_engram_site(k, T, side, true);
                ND_HIP(hipEventRecord(ev_site[k], side));
                sent[k] = true;
            }
    };
    send_sites(1);

    const int G = c.heads / c.kvheads;
    int maxlen = 0;
    for (int t = 0; t < T; ++t) maxlen = std::max(maxlen, hparams.p[t].length);
    auto layer_sites = [&](int l, int *sites) {  // waits for their engram work
        int ns = 0;
        for (int k = 0; k < c.num_sites; ++k)
            if (c.sites[k] == l) {
                ND_CHECK(sent[k], "internal: engram site joined before it was sent");
                sites[ns++] = k;
                ND_HIP(hipStreamWaitEvent(s, ev_site[k], 0));
            }
        return ns;
    };
    // int8 projections of one group of 128 or 256 positions take their input
    // prepared by the kernel that writes it (the mixing / post kernel for
    // Q|K|V|gate, the attention or gate kernel for the out-projection)
    auto target = [&](const Projection &p, PrepTarget &pt) {
        pt = PrepTarget{};
        return p.prep_target(pt, T);
    };
    bool qkvg_prepared = false;  // layer l's Q|K|V|gate input was prepared by the kernel that wrote z
    bool qkvg_done = false;      // layer l's Q|K|V|gate ran inside the previous post launch
    // the state buffers the kernels read (x, u, bx, hpost): a fused Q|K|V|gate post writes the other copy
    EngineBufs cur = b;
    float *other[4] = {alt_x, alt_u, alt_bx, alt_hpost};
    for (int l = 0; l < c.layers; ++l) {
        if (l == 0 && fuse) {  // the lanes' start, layer 0's projections and mixing (and Q|K|V|gate) in one launch
            int sites[kEngMaxSites];
            const int ns = layer_sites(0, sites);
            const int first[3] = {0, 0, 0};
            PrepTarget pt;
            qkvg_prepared = target(qkvg[0], pt);
            QkvgFused qf = qfused[0];
            const bool with_qkvg = T == 1 && !qkvg_prepared && qf.wgs > 0;
            qf.x_out = cur.x;  // (nothing in this launch reads the state it writes)
            qf.u_out = cur.u;
            qf.bx_out = cur.bx;
            qf.hpost_out = cur.hpost;
            launch_eng_post_mix(cur, layer[0], layer[0], mh, -1, phi, first, sites, ns, dims, T, pt,
                                with_qkvg ? &qf : nullptr, embed_z.p, s, er);
            qkvg_done = with_qkvg;
        }
        if (!fuse) {
            mhc_proj[l].run(s, T);
            {
                const int first[3] = {l * mhc_rows[0], l * mhc_rows[1], l * mhc_rows[2]};
                launch_eng_dense3(phi, first, mhc_rows, b.mhc_out, dims.mhc_stride, c.lanes * c.dim, b.nx, T, s);
            }
            int sites[kEngMaxSites];
            const int ns = layer_sites(l, sites);
            PrepTarget pt;
            qkvg_prepared = target(qkvg[l], pt);
            launch_eng_mix(cur, layer[l], mh, l, mhc_row[l].data(), sites, ns, dims, T, pt, s);
        }
        if (!qkvg_done) qkvg[l].run(s, T, qkvg_prepared);
        qkvg_done = false;
        PrepTarget ot;
        bool o_prepared = target(oproj[l], ot);
        // one token: norms, RoPE, the KV store (fp32, or the int8 quantiser) and attention in one kernel;
        // a chunk stores every token's K / V before any token attends; the attention prepares the
        // out-projection's input when a kv head's outputs are one group and no activation quantiser
        // runs between
        if (o_prepared && (abits || ot.group != G * HD || ot.dev != c.heads * HD)) {
            o_prepared = false;
            ot = PrepTarget{};
        }
        if (T > 1) launch_eng_qk(cur, layer[l], kv[l], dp, dims, T, s);
        const OutProj &op = ofused[l];
        EngineDims pd = dims;  // the post's view: the attention's out-projection terms, or proj
        pd.ogroups = op.codes ? c.kvheads : 0;
        launch_eng_attn_fused(cur, layer[l], kv[l], dp, hparams.p[0], maxlen, T > 1, dims, T, attn_scores.p,
                              attn_scores.n, mh, l, ot, op, s);
        if (!op.codes) {
            launch_eng_quantize(b.att, c.heads * HD, c.heads * HD, abits, T, s);
            oproj[l].run(s, T, o_prepared);
        }
        if (fuse && l + 1 < c.layers) {
            int sites[kEngMaxSites];
            const int ns = layer_sites(l + 1, sites);
            const int first[3] = {(l + 1) * mhc_rows[0], (l + 1) * mhc_rows[1], (l + 1) * mhc_rows[2]};
            PrepTarget pt;
            qkvg_prepared = target(qkvg[l + 1], pt);
            QkvgFused qf = qfused[l + 1];
            if (T == 1 && !qkvg_prepared && qf.wgs > 0) {
                qf.x_out = other[0];
                qf.u_out = other[1];
                qf.bx_out = other[2];
                qf.hpost_out = other[3];
                launch_eng_post_mix(cur, layer[l], layer[l + 1], mh, l, phi, first, sites, ns, pd, T, pt, &qf, nullptr,
                                    s);
                std::swap(cur.x, other[0]);
                std::swap(cur.u, other[1]);
                std::swap(cur.bx, other[2]);
                std::swap(cur.hpost, other[3]);
                qkvg_done = true;
            } else {
                launch_eng_post_mix(cur, layer[l], layer[l + 1], mh, l, phi, first, sites, ns, pd, T, pt, nullptr,
                                    nullptr, s);
            }
        } else {
            // (the last layer's post also computes the final norm)
            launch_eng_post(cur, layer[l], l, l + 1 < c.layers, pd, T, l + 1 == c.layers ? dptr[final_norm()] : nullptr,
                            s);
        }
        send_sites(l + 3);  // two layers ahead of their use
    }
}

void GpuEngine::step(int token, float *logits_out, float *hidden_out) {
    const int D = c.dim;
    if (token < 0 || token >= c.vocab) throw Error("token outside vocabulary");
    if (!c.window && position >= capacity) throw Error("maximum context reached");
    set_token(0, token);
    run(1);
    hipStream_t s = stream;
    if (logits_out) {
        launch_eng_quantize(b.zf, D, D, abits, 1, s);
        lm_head_host.run(s, 1);  // the GEMV stores the logits in pinned host memory
    }
    if (hidden_out) {
        hhidden.reserve(size_t(c.layers) * D);
        ND_HIP(hipMemcpyAsync(hhidden.p, b.hidden, size_t(c.layers) * D * sizeof(float), hipMemcpyDeviceToHost, s));
    }
    wait_stream(s);
    if (logits_out) std::memcpy(logits_out, hstep.p, size_t(c.vocab) * sizeof(float));
    if (hidden_out) std::memcpy(hidden_out, hhidden.p, size_t(c.layers) * D * sizeof(float));
    ++position;
}

// engine.cpp:1045-1301: the prompt in chunks of `chunk` tokens, every token's
// layers in the same launches; logits of every token, or of the last one only,
// and the last token's per-layer hidden states.
void GpuEngine::prefill(const int *tokens, int num_tokens, bool last_only, float *logits_out, float *hidden_out) {
    if (num_tokens <= 0) return;
    for (int i = 0; i < num_tokens; ++i)
        if (tokens[i] < 0 || tokens[i] >= c.vocab) throw Error("token outside vocabulary");
    if (!c.window && position + num_tokens > capacity) throw Error("maximum context reached");
    const int D = c.dim, V = c.vocab;
    hipStream_t s = stream;
    for (int c0 = 0; c0 < num_tokens; c0 += chunk) {
        const int T = std::min(chunk, num_tokens - c0);
        const bool final_chunk = c0 + T == num_tokens;
        for (int t = 0; t < T; ++t) set_token(t, tokens[c0 + t]);
        run(T);
        float *dst = nullptr;
        int rows = 0;
        if (logits_out && !last_only) {
            launch_eng_quantize(b.zf, D, D, abits, T, s);
            lm_head.run(s, T);
            dst = logits_out + size_t(c0) * V;
            rows = T;
        } else if (logits_out && final_chunk) {  // the last token only, through token 0's LM-head jobs
            if (T > 1)
                ND_HIP(hipMemcpyAsync(b.zf, b.zf + size_t(T - 1) * D, size_t(D) * sizeof(float),
                                      hipMemcpyDeviceToDevice, s));
            launch_eng_quantize(b.zf, D, D, abits, 1, s);
            lm_head.run(s, 1);
            dst = logits_out;
            rows = 1;
        }
        if (dst) {
            hlogits.reserve(size_t(chunk) * V);
            ND_HIP(hipMemcpyAsync(hlogits.p, logits.p, size_t(rows) * V * sizeof(float), hipMemcpyDeviceToHost, s));
        }
        if (final_chunk && hidden_out) {
            hhidden.reserve(size_t(c.layers) * D);
            ND_HIP(hipMemcpyAsync(hhidden.p, b.hidden + size_t(T - 1) * c.layers * D,
                                  size_t(c.layers) * D * sizeof(float), hipMemcpyDeviceToHost, s));
        }
        // the reference leaves the last token's embedding row in z (engine.cpp:1074-1075),
        // which project_candidates reads next
        ND_HIP(hipMemcpyAsync(b.zf, embed_z.p + size_t(T - 1) * D, size_t(D) * sizeof(float),
                              hipMemcpyDeviceToDevice, s));
        ND_HIP(hipStreamSynchronize(s));
        if (dst) std::memcpy(dst, hlogits.p, size_t(rows) * V * sizeof(float));
        if (final_chunk && hidden_out) std::memcpy(hidden_out, hhidden.p, size_t(c.layers) * D * sizeof(float));
        position += T;
    }
}

// engine.cpp:1302-1349: the final hidden state of the last step, quantised,
// through the LM head's candidate rows.
void GpuEngine::project_candidates(const int *candidates, int count, float *out) {
    ND_CHECK(candidates && count > 0, "candidates must be nonempty");
    for (int i = 0; i < count; ++i)
        ND_CHECK(candidates[i] >= 0 && candidates[i] < c.vocab, "candidate outside vocabulary");
    if (!out) return;
    hipStream_t s = stream;
    launch_eng_quantize(b.zf, c.dim, c.dim, abits, 1, s);
    st.hids.reserve(count);
    st.ids.reserve(count);
    st.y.reserve(count);
    st.hy.reserve(count);
    std::memcpy(st.hids.p, candidates, size_t(count) * sizeof(int32_t));
    ND_HIP(hipMemcpyAsync(st.ids.p, st.hids.p, size_t(count) * sizeof(int32_t), hipMemcpyHostToDevice, s));
    const Mat &head = mats[0];
    if (head.cq) {
        const Candidates cand = gather_candidates(*head.cq, st, st.ids.p, count, s);
        if (cand.full) {
            lm_head.run(s, 1);
            launch_gather_outputs(logits.p, c.vocab, st.ids.p, count, 1, st.y.p, s);
        } else if (head.int8) {  // engine.cpp:1312-1323: prepare once, then the candidate rows
            const Matrix &m = *head.cq;
            st.q.reserve(m.dev / 4);
            st.xs.reserve(m.groups);
            st.rot.reserve(m.dev);
            if (!launch_sdot_prepare(b.zf, nullptr, 1, 1, m.in, m.padded, m.dev, m.group, m.scale, m.kind, st.q.p,
                                     st.xs.p, nullptr, s)) {
                m.transform(b.zf, m.in, st.rot.p, 1, st.big, s);
                launch_sdot_quantize(st.rot.p, m.dev, 1, m.padded, m.dev, m.group, m.kind, st.q.p, st.xs.p, s);
            }
            const SdotJob job{cand.codes, cand.norms, st.q.p, st.xs.p, st.y.p, count, cand.n_pad, 0, 1, st.xs.p};
            launch_sdot_gemv(sdot_geom_of(m), job, nullptr, 0, cand.n_pad / kRowsPerBlock, 1, s);
        } else {
            matrix_gemv(*head.cq, st, cand.codes, cand.norms, count, cand.n_pad, b.zf, st.y.p, 1, s);
        }
    } else {
        lm_head.run(s, 1);
        launch_gather_outputs(logits.p, c.vocab, st.ids.p, count, 1, st.y.p, s);
    }
    ND_HIP(hipMemcpyAsync(st.hy.p, st.y.p, size_t(count) * sizeof(float), hipMemcpyDeviceToHost, s));
    ND_HIP(hipStreamSynchronize(s));
    std::memcpy(out, st.hy.p, size_t(count) * sizeof(float));
}

}  // namespace nd

using namespace nd;

extern "C" {

// needle2/csrc/engine.cpp:1499-1548: the same entry points and error channel.
const char *needle2_engine_error(void) { return engine_error.c_str(); }

void *needle2_engine_create(const void *config, const void *tensors, int count, int threads, int activation_bits) {
    (void)threads;
    try {
        if (!config || !tensors) throw Error("engine: null configuration or tensor table");
        return new GpuEngine(*static_cast<const EngineConfigC *>(config), static_cast<const TensorDescC *>(tensors),
                             count, activation_bits);
    } catch (const std::exception &e) {
        engine_error = e.what();
        return nullptr;
    }
}

void needle2_engine_destroy(void *p) { delete static_cast<GpuEngine *>(p); }

// The reference's projection lookup modes are CPU summation schemes; every mode runs the GPU GEMV.
void needle2_engine_set_lookup(void *, int) {}

// engine.cpp:1506-1509: the int8 matmul path, which the GPU runs everywhere.
int needle2_engine_set_sdot(void *p) {
    try {
        static_cast<GpuEngine *>(p)->set_sdot();
        return 0;
    } catch (const std::exception &e) {
        engine_error = e.what();
        return -1;
    }
}

void needle2_engine_reset(void *p, int prefix) {
    try {
        static_cast<GpuEngine *>(p)->reset(prefix);
    } catch (const std::exception &e) {
        engine_error = e.what();
    }
}

int needle2_engine_cache_prefix(void *p) {
    try {
        static_cast<GpuEngine *>(p)->cache_prefix();
        return 0;
    } catch (const std::exception &e) {
        engine_error = e.what();
        return -1;
    }
}

int needle2_engine_reset_to_prefix(void *p) {
    try {
        return static_cast<GpuEngine *>(p)->reset_to_prefix();
    } catch (const std::exception &e) {
        engine_error = e.what();
        return -1;
    }
}

int needle2_engine_step(void *p, int token, float *logits, float *hidden) {
    try {
        static_cast<GpuEngine *>(p)->step(token, logits, hidden);
        return 0;
    } catch (const std::exception &e) {
        engine_error = e.what();
        return -1;
    }
}

int needle2_engine_prefill(void *p, const int *tokens, int num_tokens, int last_only, float *logits, float *hidden) {
    try {
        static_cast<GpuEngine *>(p)->prefill(tokens, num_tokens, last_only != 0, logits, hidden);
        return 0;
    } catch (const std::exception &e) {
        engine_error = e.what();
        return -1;
    }
}

int needle2_engine_step_candidates(void *p, int token, const int *candidates, int num_candidates,
                                   float *candidate_logits, float *hidden) {
    try {
        auto *e = static_cast<GpuEngine *>(p);
        ND_CHECK(candidates && num_candidates > 0, "candidates must be nonempty");
        for (int i = 0; i < num_candidates; ++i)
            ND_CHECK(candidates[i] >= 0 && candidates[i] < e->c.vocab, "candidate outside vocabulary");
        e->step(token, nullptr, hidden);
        e->project_candidates(candidates, num_candidates, candidate_logits);
        return 0;
    } catch (const std::exception &e) {
        engine_error = e.what();
        return -1;
    }
}

int needle2_engine_project_candidates(void *p, const int *candidates, int num_candidates, float *candidate_logits) {
    try {
        static_cast<GpuEngine *>(p)->project_candidates(candidates, num_candidates, candidate_logits);
        return 0;
    } catch (const std::exception &e) {
        engine_error = e.what();
        return -1;
    }
}

int needle2_engine_decode_loop(void *p, int first_token, int max_new_tokens, const void *dfa, int *output_tokens,
                               int *generated) {
    try {
        return static_cast<GpuEngine *>(p)->decode_loop(first_token, max_new_tokens, static_cast<const DfaC *>(dfa),
                                                        output_tokens, generated);
    } catch (const std::exception &e) {
        engine_error = e.what();
        return -1;
    }
}

int needle2_engine_import(void *p, int position, int pinned, const int *ids, const int *positions, int count,
                          const float *k, const float *v) {
    try {
        static_cast<GpuEngine *>(p)->import_state(position, pinned, ids, positions, count, k, v);
        return 0;
    } catch (const std::exception &e) {
        engine_error = e.what();
        return -1;
    }
}

int needle2_engine_set_int8_kv(void *p, int enable) {
    try {
        auto *e = static_cast<GpuEngine *>(p);
        e->int8_kv = enable != 0;
        e->reset(e->prefix);
        return 0;
    } catch (const std::exception &e) {
        engine_error = e.what();
        return -1;
    }
}

size_t needle2_engine_kv_storage_bytes(void *p) { return static_cast<GpuEngine *>(p)->kv_storage_bytes(); }

}  // extern "C"
