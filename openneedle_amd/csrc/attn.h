// int8 KV cache: device argument blocks and launchers (attn_kernels.hip).
#pragma once

#include "common.h"

namespace nd {

// Quantize `count` tokens per sequence into one layer of the cache.
// k, v: fp32 [seqs][count][kvheads][head_dim]; token i of sequence s goes to
// slot first_slot[s] + i (device array, checked against capacity by the host).
struct KvStoreArgs {
    const float *k, *v;
    int8_t *k8, *v8;       // layer base, [seq][kvh][capacity][head_dim]
    float *ks, *vs;        // layer base, [seq][kvh][capacity]
    const int *first_slot;
    int seqs, count, kvheads, head_dim, capacity;
};

// Decode attention for one layer. q, out: fp32 [seqs][kvheads * G][head_dim].
// Sequence s attends slots[j] (or j when slots is null) for j < its length
// (lengths[s], or `length` when lengths is null; never more than `length`);
// a listed slot outside [0, capacity) is skipped.
// The slot range is cut into `splits` pieces of slots_per_split; with more
// than one split, per-split records go to part and a merge pass writes out.
struct AttnArgs {
    int8_t *k8, *v8;       // the layer's cache (read; written only for new_k / new_v)
    float *ks, *vs;
    const float *q;
    float *out;
    float *part;           // [seqs * heads][splits][head_dim + 2]
    const int *slots;      // nullable, device
    const int *lengths;    // nullable, device
    int seqs, kvheads, head_dim, capacity, length, splits, slots_per_split;
    float scale;           // 1/sqrt(head_dim), computed on the host like the reference
    int slots_stride;      // sequence s's list starts at slots + s * slots_stride (0: one shared list)
    int shared_cache;      // nonzero: every sequence reads the same [kvheads][capacity] cache (the
                           // tokens of one prompt chunk, each with its own slot list)
    PrepOut prep;          // q set (one split, heads * head_dim a multiple of 64): out is also left
                           // prepared as the next int8 projection's input, sequence = batch row
    const float *new_k, *new_v;  // non-null (no slot list, no shared cache): one new token per sequence
    const int *new_slot;         // ([seqs][kvheads][head_dim]) is first stored at new_slot[seq]
};

bool attn_supported(int head_dim, int group);
void launch_kv_store(const KvStoreArgs &a, hipStream_t s);
void launch_attention(AttnArgs a, int group, hipStream_t s);

}  // namespace nd
