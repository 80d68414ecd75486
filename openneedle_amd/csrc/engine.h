// Single-sequence decode engine on the GPU (needle2/csrc/engine.cpp:340-1044):
// device argument blocks shared by engine.cpp and engine_kernels.hip.
#pragma once

#include "common.h"

namespace nd {

constexpr int kEngMaxHalfHd = 64;  // head_dim <= 128
constexpr int kEngMaxTables = 16;  // engram tables per site
constexpr int kEngMaxSites = 4;
constexpr int kEngMaxTaps = 16;
constexpr size_t kEngScoreLds = 49152;  // bytes of fp32 attention scores kept in LDS
constexpr int kEngThreads = 1024;  // every glue kernel is one workgroup of this size

// Values of one token that depend only on its position, the token history
// and the cache geometry; the host computes them (with the reference's own
// integer hashing and std::cos / std::sin) and uploads them once per step or
// prompt chunk, one record per token.
struct StepParams {
    int position, slot;                                // this token's cache slot (engine.cpp:500)
    int length, prefix_count, start, prefix, window;   // attention slot list (engine.cpp:898-911)
    int ring;                                          // KV slots past the prefix (window models)
    int chunk_start;                                   // first position of this token's chunk
    int engram_zero[kEngMaxSites];                     // bit t: table t of site s reads zeros
    int tap_pos[kEngMaxTaps];                          // position read by each conv tap, -1: skipped
    float rope_cos[kEngMaxHalfHd], rope_sin[kEngMaxHalfHd];
};

// A decode step's slot-list parameters (StepParams' first fields), passed by
// value to the attention launch: in its kernel arguments they arrive with the
// first round of argument loads, a memory round trip ahead of the uploaded
// StepParams.
struct StepHead {
    int slot, length, prefix_count, start, prefix, window, ring;
};

// Work buffers hold a chunk of tokens: token t of a launch is blockIdx.y and
// its vectors sit t per-token sizes past the token-0 pointers below.
// Prompt chunk: at most kEngMaxChunk tokens (engine.cpp:1054 takes 32), every
// token of a chunk in the same launches; a window model's chunk is at most its
// window, and long contexts take a shorter chunk (down to 32) that holds the
// attention-score buffer (chunk * kv heads * G * max length floats) to
// kEngScoreBudget bytes.
constexpr int kEngMaxChunk = 256;
constexpr int kEngMinChunk = 32;
constexpr size_t kEngScoreBudget = size_t(512) << 20;

struct EngineDims {
    int D, N, H, KV, HD, A, K, hada, layers, tables, subdim, taps, capacity, engring, abits;
    int sites;       // engram sites (per-token stride of ek / ev: sites * D)
    int mhc_stride;  // per-token stride of each mhc_out buffer
    float sqrt_d;    // std::sqrt(float(D)) (engine.cpp:974, 987)
    float inv_hada;  // 1 / std::sqrt(float(hada)), the Hadamard normalisation
    float scale;     // 1 / std::sqrt(float(head_dim)) (engine.cpp:914)
    int ogroups;     // > 0: the post adds these out-projection terms per row (oparts) instead of reading proj
};

// Layer parameters (device pointers into the engine's fp32 copies of the
// dense tensors; the matrices run through the GEMV kernels).
struct LayerDev {
    const float *norm_in, *q_norm, *k_norm, *post_norm, *attn_gate, *pre_hada, *d1, *d2, *d3;
};

// The mHC scalars and vectors of the model (engine.cpp:980-984, 1036).
struct MhcDev {
    const float *a_pre, *a_post, *a_res, *b_pre, *b_post, *b_res;
};

// Work buffers (device), token 0's vectors; token t's are t per-token sizes
// further (EngineDims): x, nx N*D; u, bx, z, proj, e, rawv, zf D; q, gate,
// att A; k, v K; hidden layers*D; hpre, hpost N; hres, hroute N*N; mhc_out
// mhc_stride; ek, ev sites*D; slots capacity. The engram ring is shared.
struct EngineBufs {
    float *x, *nx, *u, *bx, *z, *q, *k, *v, *gate, *att, *proj, *hidden;
    float *hpre, *hpost, *hres;     // mixed gates (N, N, N*N)
    float *hroute;                  // Sinkhorn of the layer's residual routing logits (N*N)
    float *mhc_out[3];              // raw mHC projections of the layer (pre, post, res rows)
    float *e, *ek, *ev, *rawv;      // engram rows [D], keys [sites][D], values [sites][D], raw values [D]
    float *engring;                 // [sites][engring][D], row = position % engring
    float *zf;                      // final hidden, input of the LM head
    int *slots;                     // attention slot list
    float *oparts;                  // out-projection terms [KV][D] (the attention's, see OutProj)
};

// The out-projection inside the attention launch, for an FP32 CQ matrix whose
// groups of 128 input positions are the G query heads of one kv head (the
// released geometry's G * head_dim = 128): the input's FWHT and every row's
// group sum split by group, so kv head h's workgroup computes, for every
// output row, the term p_h = gd_h * half(norm_h) of its own group (the GEMV
// kernels' arithmetic and order: gd_h sums cb * rot over the group's
// positions in order) into parts[token][h][row], and the post kernel adds
// the terms in group order, sum = ((0 + p_0) + p_1) + ... as the GEMV does:
// the same bits as the separate out-projection launch.
struct OutProj {
    const uint4 *codes;     // the matrix's device layout (null: no fused out-projection)
    const uint16_t *norms;
    float *parts;           // [tokens][kv heads][rows]
    int rows, chunks, groups, kind;
    float scale;            // 1 / sqrt(128)
    float lut[16];
    // one token with the scores in LDS: 2^split_shift workgroups per kv head, each running the head's
    // attention (the same arithmetic) and a contiguous share of the rows; part 0 stores the outputs
    int split_shift;
};

// Rows of the fused Q|K|V|gate projection per workgroup (512 threads: four per row, one per group)
#ifndef ND_QKVG_ROWS
#define ND_QKVG_ROWS 128
#endif
constexpr int kQkvgRows = ND_QKVG_ROWS;
static_assert(kQkvgRows == 64 || kQkvgRows == 128, "slices of 64 or 128 rows");

// The next layer's Q|K|V|gate projection inside the fused post / mixing
// launch of one token, for FP32 CQ matrices of 2- or 4-bit codes in groups of
// 128 over d_model <= 512 inputs: every workgroup runs the post and mixing
// (the same arithmetic, so every workgroup holds the same z), then one slice
// of kQkvgRows rows of one piece with the GEMV kernels' arithmetic and order
// (the input's FWHT per group, the product table, gd_g summed over the
// group's codes in order, sum = ((0 + p_0) + p_1) + ... with p_g = gd_g *
// half(norm_g)): the separate launch's bits. Workgroup 0 alone stores the
// layer state, into the *_out buffers (the other workgroups may still be
// reading the inputs), which the host then takes as the current ones.
struct QkvgPiece {
    const uint4 *codes;
    const uint16_t *norms;
    float *y;            // the piece's outputs (token 0)
    int rows, sub_begin;  // rows; first workgroup of the piece (one per kQkvgRows rows)
};
struct QkvgFused {
    QkvgPiece piece[4];
    int pieces, wgs;  // wgs: workgroups of all pieces (0: not fused)
    int chunks, groups, kind;
    float scale;      // 1 / sqrt(128)
    float lut[16];
    float *x_out, *u_out, *bx_out, *hpost_out;  // the new lanes, u, bx and lane post gates
};

// The tokens' embedding rows decoded inside the first layer's launch (a CQ
// embedding whose padded width is d_model): the row kernel's arithmetic
// (cb[code] * half(norm)), then the FWHT of each group in the transform's
// stage order and the scale, into z[t][d_model] as the row kernels leave it.
struct EmbedRows {
    const uint4 *codes;  // null: the rows come from z, decoded by the row kernels
    const uint16_t *norms;
    const int64_t *ids;  // the tokens' rows
    float *z;
    CqGeom g;
};

// KV cache of one layer: fp32 (k32 / v32) or int8 codes with fp32 scales,
// [kvheads][capacity][head_dim] (scales [kvheads][capacity]).
struct KvLayer {
    float *k32, *v32;
    int8_t *k8, *v8;
    float *ks, *vs;
};

// The int8 path's prepared input of the projection that reads a kernel's
// output (the q / xs / xst buffers its prepare launch would fill, see
// launch_sdot_prepare): a kernel given a target with q set prepares token t's
// row itself, one wave per group of 128 or 256 positions, in the same
// arithmetic. xst is null for one token, else [groups][tokens].
struct PrepTarget {
    int8_t *q;   // [tokens][dev] permuted codes (null: nothing to prepare)
    float *xs;   // [tokens][groups]
    float *xst;
    int dev, padded, groups, kind, group;
    float scale;
};

// Every launcher runs `tokens` tokens (blockIdx.y), with p the device array of their StepParams.
void launch_eng_start(const float *z, const EngineBufs &b, const EngineDims &d, int tokens, hipStream_t s);
void launch_eng_engram_in(const EngineBufs &b, const StepParams *p, int site, const EngineDims &d, int tokens,
                          hipStream_t s);
// the dilated conv of every token (in-chunk taps read the chunk's raw values),
// then the ring rows of the chunk's last positions
void launch_eng_engram_out(const EngineBufs &b, const float *taps, const StepParams *p, int site,
                           const EngineDims &d, int tokens, hipStream_t s);
// mixing, engram gates and the attention input of layer l; mhc_row[m] is the
// first row of the layer inside b.mhc_out[m]; sites: engram sites at this layer
// (pt: the Q|K|V|gate projection's int8 input, prepared from z)
void launch_eng_mix(const EngineBufs &b, const LayerDev &ld, const MhcDev &mh, int l, const int *mhc_row,
                    const int *sites, int nsites, const EngineDims &d, int tokens, const PrepTarget &pt,
                    hipStream_t s);
// q / k norms, RoPE and the K / V store of every token
void launch_eng_qk(const EngineBufs &b, const LayerDev &ld, const KvLayer &kv, const StepParams *p,
                   const EngineDims &d, int tokens, hipStream_t s);
// Attention + output gate of every kv head over an fp32 or int8 KV cache (kv.k8 set); with `prepared`
// false (one token) it also does that token's norms, RoPE and KV store, else eng_qk did. scores: null
// when G * max_length floats fit kEngScoreLds, else a device buffer of tokens * kvheads * G * max_length
// floats (scores_n, checked). It also runs layer l's residual routing (Sinkhorn of hres into hroute) in one more workgroup
// per token, and prepares the out-projection's int8 input from att when pt.q is set (a group of one kv
// head's outputs, heads / kvheads * head_dim positions).
// With op.codes set (and G * head_dim == 128, no pt) each kv head's workgroup also computes its group's
// out-projection terms (OutProj).
// hp: the host copy of token 0's StepParams (a step's slot list goes in the kernel arguments).
void launch_eng_attn_fused(const EngineBufs &b, const LayerDev &ld, const KvLayer &kv, const StepParams *p,
                           const StepParams &hp, int max_length, bool prepared, const EngineDims &d, int tokens,
                           float *scores, size_t scores_n, const MhcDev &mh, int l, const PrepTarget &pt,
                           const OutProj &op, hipStream_t s);
// K / V rows [count][kvheads][head_dim] into cache slots[count] (device) of one layer
void launch_eng_kv_import(const float *k, const float *v, const int *slots, int count, const KvLayer &kv,
                          const EngineDims &d, hipStream_t s);
// final_norm (the last layer; null: none): also zf = rms(hidden) * (1 + final_norm)
void launch_eng_post(const EngineBufs &b, const LayerDev &ld, int l, bool next_rms,
                     const EngineDims &d, int tokens, const float *final_norm, hipStream_t s);
// The post of layer l, then layer l + 1's dense mHC projections (rows first[m] .. of the three
// matrices w[m]) and mixing with the engram sites[0..nsites), in one launch; only where
// eng_post_mix_fits(d). qf (null: none): layer l + 1's Q|K|V|gate projection in the same launch
// (QkvgFused; one token, no activation quantiser, no int8 target). start (l = -1):
// no post; the lanes come from the tokens' embedding rows start[t][D] (launch_eng_start's work; er.codes
// set: decoded here into start, EmbedRows), then layer 0's projections and mixing.
bool eng_post_mix_fits(const EngineDims &d);
void launch_eng_post_mix(const EngineBufs &b, const LayerDev &ld, const LayerDev &ldn, const MhcDev &mh, int l,
                         const float *const *w, const int *first, const int *sites, int nsites, const EngineDims &d,
                         int tokens, const PrepTarget &pt, const QkvgFused *qf, const float *start, hipStream_t s,
                         const EmbedRows &er = EmbedRows{});
// x[t][0..n) for t < tokens, rows `stride` apart
void launch_eng_quantize(float *x, int n, int stride, int bits, int tokens, hipStream_t s);
// y[t][r] = dot(W[first + r], x[t]) over cols for r < rows (dense fp32 matrices); x rows cols
// apart, y rows ystride apart
void launch_eng_dense(const float *w, int cols, int first, int rows, const float *x, float *y, int ystride,
                      int tokens, hipStream_t s);
// y[m][t][r] = dot(W_m[first[m] + r], x[t]) for r < rows[m], m < 3 (a null W_m is skipped), one
// launch; y rows ystride apart
void launch_eng_dense3(const float *const *w, const int *first, const int *rows, float *const *y, int ystride,
                       int cols, const float *x, int tokens, hipStream_t s);
// y[i][:] = W[ids[i]][:] (dense row copy)
void launch_eng_dense_rows(const float *w, int cols, const int64_t *ids, int count, float *y, hipStream_t s);

}  // namespace nd
