/*
 * CPU restatement of OpenNeedle's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP kernels
 * in openneedle_amd/ are compared against. Only tests/, the smoke check and
 * the CPU-baseline leg of bench.py may load it; product code never does.
 *
 * Every function restates the x86 (non-NEON) branch of the reference, with
 * the operation order kept so the results are bit-identical to the reference
 * compiled with its own flags (-O3 -std=c++17, which disables FP
 * contraction). Build with -ffp-contract=off.
 *
 * Pins (tests/test_oracle.py): each function is checked against the
 * reference built from source (oracle/_ref, bit-exact), against closed forms
 * (dense Sylvester-Hadamard, integer dot products, fp64 softmax) and against
 * the reference's own known-answer tests.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* needle2/csrc/cq.cpp:14-28 (portable branch): exact IEEE binary16 -> binary32. */
float nd_half_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 31u, mantissa = h & 1023u, bits;
    if (exponent == 0) {
        if (mantissa == 0) {
            bits = sign;
        } else {
            int e = -14;
            while (!(mantissa & 1024u)) { mantissa <<= 1; --e; }
            bits = sign | (uint32_t)(e + 127) << 23 | (mantissa & 1023u) << 13;
        }
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112) << 23) | (mantissa << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* needle2/csrc/cq.cpp:30-46: in-place normalized Walsh-Hadamard transform.
 * Butterfly stages h = 1, 2, 4, ... with (a+b, a-b), then a multiply by the
 * float 1/sqrt(n). The stage order is what makes the result bit-exact. */
void nd_hadamard(float *v, int n)
{
    for (int h = 1; h < n; h *= 2)
        for (int base = 0; base < n; base += 2 * h)
            for (int j = 0; j < h; ++j) {
                float a = v[base + j], b = v[base + j + h];
                v[base + j] = a + b;
                v[base + j + h] = a - b;
            }
    float scale = 1.0f / sqrtf((float)n);
    for (int i = 0; i < n; ++i) v[i] *= scale;
}

/* needle2/csrc/cq.cpp:48-53: code i of an LSB-first bitstream. */
unsigned nd_index_at(const uint8_t *p, int i, int bits)
{
    int bit = i * bits, byte = bit >> 3, shift = bit & 7;
    unsigned word = p[byte];
    if (shift + bits > 8) word |= (unsigned)p[byte + 1] << 8;
    return (word >> shift) & ((1u << bits) - 1);
}

typedef struct {
    const uint8_t *packed;
    const uint16_t *norms;
    int out, in, bits, group, padded, groups, rowbytes, storage_bits;
    float cb[16];
} nd_cq;

/* needle2/csrc/cq.cpp:61-70 (geometry) and 71-74 (ternary crumb mapping). */
static void nd_cq_init(nd_cq *q, const uint8_t *packed, const uint16_t *norms,
                       int out, int in, int bits, int group, const float *cb)
{
    q->packed = packed;
    q->norms = norms;
    q->out = out;
    q->in = in;
    q->bits = bits;
    q->group = group;
    q->padded = (in + group - 1) / group * group;
    q->groups = q->padded / group;
    q->storage_bits = bits == 5 ? 2 : bits;
    q->rowbytes = q->padded * q->storage_bits / 8;
    memset(q->cb, 0, sizeof q->cb);
    memcpy(q->cb, cb, sizeof(float) * (size_t)(bits == 5 ? 3 : 1 << bits));
}

static float nd_weight(const nd_cq *q, const uint8_t *p, int i)
{
    unsigned idx = nd_index_at(p, i, q->storage_bits);
    /* Ternary crumb 2 is rejected by the Python loader; read it as zero. */
    if (q->bits == 5) return idx == 3 ? q->cb[0] : idx == 2 ? 0.0f : q->cb[idx + 1];
    return q->cb[idx];
}

/* needle2/csrc/cq.cpp:153-156: copy, zero-pad, FWHT per group. */
static void nd_transform(const nd_cq *q, const float *x, float *rot)
{
    memcpy(rot, x, sizeof(float) * (size_t)q->in);
    for (int i = q->in; i < q->padded; ++i) rot[i] = 0.0f;
    for (int g = 0; g < q->groups; ++g) nd_hadamard(rot + (size_t)g * q->group, q->group);
}

/* needle2/csrc/cq.cpp:75-109 (x86 tail): sequential sum of weight*x. */
static float nd_group_dot(const nd_cq *q, const uint8_t *p, const float *x)
{
    float sum = 0.0f;
    for (int i = 0; i < q->group; ++i) sum += nd_weight(q, p, i) * x[i];
    return sum;
}

/* needle2/csrc/cq.cpp:165-197: y[b][r] = sum_g group_dot * half(norm), sequential
 * over g. The token-pair branch (group_dot_pair) has the same per-token order,
 * so every batch row is computed like batch 1. Returns 0, or -1 on OOM. */
int nd_cq_linear(const uint8_t *packed, const uint16_t *norms, int out, int in, int bits,
                 int group, const float *cb, const float *x, float *y, int batch, int threads)
{
    nd_cq q;
    nd_cq_init(&q, packed, norms, out, in, bits, group, cb);
    float *rot = (float *)malloc(sizeof(float) * (size_t)(batch > 0 ? batch : 1) * q.padded);
    if (!rot) return -1;
    for (int b = 0; b < batch; ++b) nd_transform(&q, x + (size_t)b * in, rot + (size_t)b * q.padded);
    int gbytes = group * q.storage_bits / 8;
#pragma omp parallel for num_threads(threads) if (threads > 1) schedule(static)
    for (int r = 0; r < out; ++r) {
        const uint8_t *p = packed + (size_t)r * q.rowbytes;
        const uint16_t *s = norms + (size_t)r * q.groups;
        for (int b = 0; b < batch; ++b) {
            const float *rb = rot + (size_t)b * q.padded;
            float sum = 0.0f;
            for (int g = 0; g < q.groups; ++g)
                sum += nd_group_dot(&q, p + (size_t)g * gbytes, rb + (size_t)g * group) * nd_half_float(s[g]);
            y[(size_t)b * out + r] = sum;
        }
    }
    free(rot);
    return 0;
}

/* needle2/csrc/cq.cpp:276-284: dequantize row r (cb*norm, then FWHT), cropped to in. */
int nd_cq_rows(const uint8_t *packed, const uint16_t *norms, int out, int in, int bits,
               int group, const float *cb, const int64_t *ids, float *y, int count)
{
    nd_cq q;
    nd_cq_init(&q, packed, norms, out, in, bits, group, cb);
    float *tmp = (float *)malloc(sizeof(float) * (size_t)q.padded);
    if (!tmp) return -1;
    for (int i = 0; i < count; ++i) {
        int64_t r = ids[i];
        const uint8_t *p = packed + (size_t)r * q.rowbytes;
        for (int g = 0; g < q.groups; ++g) {
            float norm = nd_half_float(norms[(size_t)r * q.groups + g]);
            for (int j = 0; j < group; ++j) tmp[g * group + j] = nd_weight(&q, p, g * group + j) * norm;
            nd_hadamard(tmp + (size_t)g * group, group);
        }
        memcpy(y + (size_t)i * in, tmp, sizeof(float) * (size_t)in);
    }
    free(tmp);
    return 0;
}

static float nd_maxf(float a, float b) { return a < b ? b : a; }              /* std::max */
static float nd_clampf(float v, float lo, float hi) { return v < lo ? lo : hi < v ? hi : v; } /* std::clamp */

/* needle2/csrc/sdot.cpp:35-45: int8 centroids and the centroid scale. */
void nd_sdot_centroids(const float *cb, int bits, int8_t *centroids, float *centroid_scale)
{
    float maximum = 0.0f;
    for (int i = 0; i < (1 << bits); ++i) maximum = nd_maxf(maximum, fabsf(cb[i]));
    float cs = maximum > 0 ? maximum / 127 : 1;
    for (int i = 0; i < (1 << bits); ++i)
        centroids[i] = (int8_t)nd_clampf(nearbyintf(cb[i] / cs), -127.0f, 127.0f);
    *centroid_scale = cs;
}

/* needle2/csrc/sdot.cpp:47-81 (scalar branch): FWHT per group, absmax,
 * scale = absmax/127 (1 when absmax == 0, absmax when the quotient underflows),
 * q = clamp(nearbyint(x/scale), +-127). q is written in natural order; the
 * reference's lane permutation (82-101) is applied to both operands of every
 * product, so it does not change any int32 dot. */
void nd_sdot_prepare(const float *x, int in, int group, int8_t *q, float *scales)
{
    int padded = (in + group - 1) / group * group;
    float *rot = (float *)malloc(sizeof(float) * (size_t)padded);
    memcpy(rot, x, sizeof(float) * (size_t)in);
    for (int i = in; i < padded; ++i) rot[i] = 0.0f;
    for (int g = 0; g < padded / group; ++g) {
        float *v = rot + (size_t)g * group;
        nd_hadamard(v, group);
        float absmax = 0.0f;
        for (int i = 0; i < group; ++i) absmax = nd_maxf(absmax, fabsf(v[i]));
        float scale = absmax > 0 ? absmax / 127 : 1;
        if (!scale) scale = absmax;
        scales[g] = scale;
        for (int i = 0; i < group; ++i)
            q[(size_t)g * group + i] = (int8_t)nd_clampf(nearbyintf(v[i] / scale), -127.0f, 127.0f);
    }
    free(rot);
}

/* needle2/csrc/sdot.cpp:108-137 (scalar branch): int32 per (row, group). */
void nd_sdot_dots(const uint8_t *packed, int out, int in, int bits, int group,
                  const int8_t *centroids, const int8_t *q, int32_t *dots)
{
    int padded = (in + group - 1) / group * group, groups = padded / group;
    int rowbytes = padded * bits / 8;
    for (int r = 0; r < out; ++r) {
        const uint8_t *p = packed + (size_t)r * rowbytes;
        for (int g = 0; g < groups; ++g) {
            int32_t sum = 0;
            for (int i = 0; i < group; ++i)
                sum += (int32_t)centroids[nd_index_at(p, g * group + i, bits)] * (int32_t)q[(size_t)g * group + i];
            dots[(size_t)r * groups + g] = sum;
        }
    }
}

/* needle2/csrc/sdot.cpp:142-149, 338-346, 356-359: per batch row prepare, then
 * value = sum_g (float(dot_g) * norm_scale[r][g]) * x_scale[g], left to right,
 * sequential over g, with norm_scale = half(norm) * centroid_scale. */
int nd_sdot_linear(const uint8_t *packed, const uint16_t *norms, int out, int in, int bits,
                   int group, const float *cb, const float *x, float *y, int batch, int threads)
{
    int padded = (in + group - 1) / group * group, groups = padded / group;
    int rowbytes = padded * bits / 8;
    int8_t centroids[16];
    float cs;
    nd_sdot_centroids(cb, bits, centroids, &cs);
    float *ns = (float *)malloc(sizeof(float) * (size_t)out * groups);
    int8_t *q = (int8_t *)malloc((size_t)padded);
    float *xs = (float *)malloc(sizeof(float) * (size_t)groups);
    if (!ns || !q || !xs) { free(ns); free(q); free(xs); return -1; }
    for (size_t i = 0; i < (size_t)out * groups; ++i) ns[i] = nd_half_float(norms[i]) * cs;
    for (int b = 0; b < batch; ++b) {
        nd_sdot_prepare(x + (size_t)b * in, in, group, q, xs);
        float *yb = y + (size_t)b * out;
#pragma omp parallel for num_threads(threads) if (threads > 1 && out >= 128) schedule(static)
        for (int r = 0; r < out; ++r) {
            const uint8_t *p = packed + (size_t)r * rowbytes;
            float value = 0.0f;
            for (int g = 0; g < groups; ++g) {
                int32_t dot = 0;
                for (int i = 0; i < group; ++i)
                    dot += (int32_t)centroids[nd_index_at(p, g * group + i, bits)] * (int32_t)q[(size_t)g * group + i];
                value += (float)dot * ns[(size_t)r * groups + g] * xs[g];
            }
            yb[r] = value;
        }
    }
    free(ns); free(q); free(xs);
    return 0;
}

/* needle2/csrc/engine.cpp:1008-1020: per (token, kv-head) absmax int8 with
 * scale = max/127 and a multiply by the reciprocal 127/max. src and dst are
 * [tokens][kvheads][head_dim]; scales are [tokens][kvheads]. */
void nd_kv_quantize(const float *src, int tokens, int kvheads, int head_dim, int8_t *dst, float *scales)
{
    for (int t = 0; t < tokens; ++t)
        for (int kh = 0; kh < kvheads; ++kh) {
            const float *p = src + ((size_t)t * kvheads + kh) * head_dim;
            int8_t *d = dst + ((size_t)t * kvheads + kh) * head_dim;
            float maximum = 0.0f;
            for (int i = 0; i < head_dim; ++i) maximum = nd_maxf(maximum, fabsf(p[i]));
            float scale = maximum > 0 ? maximum / 127.0f : 1.0f;
            float inv = maximum > 0 ? 127.0f / maximum : 0.0f;
            scales[(size_t)t * kvheads + kh] = scale;
            for (int i = 0; i < head_dim; ++i) {
                float v = nearbyintf(p[i] * inv);
                v = v < 127.0f ? v : 127.0f;      /* std::min(127, v) */
                v = -127.0f < v ? v : -127.0f;    /* std::max(-127, v) */
                d[i] = (int8_t)v;
            }
        }
}

/* needle2/csrc/engine.cpp:898-967 (int8 branch, x86 tails), 56-74, 137-147,
 * 816-897. For every head h (kv head h / (heads/kvheads)):
 *   s = dot(q_h, float(k_i8)) * k_scale, then s *= 1/sqrt(head_dim);
 *   p = exp(s - max) / sum;  out[d] = sum_s (p_s * v_scale_s) * float(v_i8[s][d]).
 * Caches are [slot][kvheads][head_dim] with scales [slot][kvheads]; slots[s]
 * lists the attended cache slots in order. Paired (GQA) heads use the same
 * per-element arithmetic on x86, so one loop covers both branches. */
int nd_attention_i8(const float *q, int heads, int kvheads, int head_dim,
                    const int8_t *keys, const int8_t *values, const float *k_scales,
                    const float *v_scales, const int *slots, int length, float *out)
{
    float *s0 = (float *)malloc(sizeof(float) * (size_t)(length > 0 ? length : 1));
    if (!s0) return -1;
    int group = heads / kvheads;
    for (int h = 0; h < heads; ++h) {
        int kh = h / group;
        const float *qh = q + (size_t)h * head_dim;
        float maximum = -INFINITY, scale = 1 / sqrtf((float)head_dim);
        for (int s = 0; s < length; ++s) {
            size_t row = (size_t)slots[s] * kvheads + kh;
            const int8_t *k = keys + row * head_dim;
            float sum = 0.0f;
            for (int d = 0; d < head_dim; ++d) sum += qh[d] * (float)k[d];
            s0[s] = sum * k_scales[row];
            s0[s] *= scale;
            maximum = nd_maxf(maximum, s0[s]);
        }
        float den = 0.0f;
        for (int s = 0; s < length; ++s) { s0[s] = expf(s0[s] - maximum); den += s0[s]; }
        float inv = 1 / den;
        for (int s = 0; s < length; ++s) s0[s] *= inv;
        for (int d = 0; d < head_dim; ++d) {
            float a = 0.0f;
            for (int s = 0; s < length; ++s) {
                size_t row = (size_t)slots[s] * kvheads + kh;
                float prob = s0[s];
                prob *= v_scales[row];
                a += prob * (float)values[row * head_dim + d];
            }
            out[(size_t)h * head_dim + d] = a;
        }
    }
    free(s0);
    return 0;
}
