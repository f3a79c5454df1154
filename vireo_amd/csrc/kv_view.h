// The device layout of a contiguous KV store, for kernels that append to it in
// place: block b of layer l at base + (l * max_blocks + b) * 2 G d (G key rows,
// then G value rows, of d floats), its running mean key at
// ksum + (l * max_blocks + b) * d.
#pragma once

struct VireoKV;

struct KvContigView {
    float *base, *ksum;
    int layers, max_blocks, G, d;  // layers: the store's (layer x kv-head) rows
};

// 0 and the view of a contiguous store; -EINVAL for any other store
int vh_kv_contig_view(const VireoKV *S, KvContigView *v);
