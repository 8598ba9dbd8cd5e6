// Host/device parameter block of the split-K decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fastdiv.h"

namespace akv {

struct DecodeParams {
    // shapes
    int B, Hq, Hkv, M, D, g, R, nchunk, prows;  // prows = min(16, R): rows per partial
    // query / hot tier (fp16)
    const _Float16 *q;
    const _Float16 *khot, *vhot;
    int64_t n_hot;
    int64_t h_stride;             // hot token rows per (b, kv-head) (>= n_hot)
    // warm tier
    const void *kc, *vc;          // packed codes
    const void *ks, *kz, *vs, *vz; // meta
    int64_t n_warm;
    int64_t w_stride;             // warm token rows per head (legacy; == n_warm for affine)
    int kc_row, vc_row;           // bytes per packed row
    int T, Gv;                    // affine: K token block, V channel group
    int tshift;                   // affine: log2(T / 32) when T / 32 is a power of two, else -1
    int64_t nblk;                 // affine: K blocks per (b, kv-head)
    int n_out;                    // affine outliers per block
    const int64_t *k_oidx, *v_oidx;
    const _Float16 *k_odata, *v_odata;
    int gs, lg, meta_dt;          // legacy: group size, groups per row, meta dtype
    int warm_heads;               // legacy: 1 or Hkv
    int legacy_sym;               // legacy: 0/1 when forced
    const int *sym_flags;         // legacy: device flags [K, V] when detected
    float half_max_k, half_max_v; // legacy: maxv // 2
    // softmax
    float scale_log2;             // sm_scale * log2(e)
    int hot_first;
    int64_t N;                    // logical tokens n_hot + n_warm
    // split schedule
    int n_wsplit, n_hsplit, nsplit;
    int64_t wsplit_len, hsplit_len;
    // outputs / workspace
    float *part;                  // split partials
    uint64_t *split_ctr;          // fast kernel: arrival counts per (b, kv-head, row chunk), a byte per XCD; null = merge
                                  // in decode_reduce_kernel / finish_kernel
    float *stash;                 // [B][Hq][M][N] raw logits q.k (or null); x * scale_log2 is the log2 domain
    float *rowstats;              // [B*Hq*M][2] (M, 1 / L): the reciprocal once per row
    _Float16 *out;                // [B][Hq][M][D]
    int out_bf16;                 // reduce only: write bf16 (chunked prefill with bf16 queries)
    float *attn_out;              // normalised weights (or null)
    float *scores;                // importance EMA (or null)
    int64_t n_scores;
    float decay;
    // fast path (decode_fast.hip): bytes of one LDS ring slot
    int slot_bytes;
    // fast path: the workgroup id split into (split, kv-head, batch x row chunk) and a
    // row of a chunk into (query head, query position) without integer division
    FastDiv fd_nsplit, fd_hkv, fd_nchunk, fd_m;
};

// Launch split + reduce (+ weights/importance) kernels.  `sym_src` = {meta dtype, count}
// of the legacy zero-point tensors when the symmetric branch must be detected.
// flags[0] (K) / flags[1] (V) = 1 iff every zero-point is 0 (the reference's symmetric branch).
hipError_t legacy_sym_launch(const void *kz, const void *vz, int64_t n, int dt, int *flags, hipStream_t s);

hipError_t decode_launch(const DecodeParams &p, int kb, int vb, int wk, const int *sym_src, hipStream_t s);

// Merge split partials (m, l, acc) into the output (and row statistics).
hipError_t decode_reduce_launch(const DecodeParams &p, hipStream_t s);

// LDS-streamed split kernel for the block-affine tier (decode_fast.hip).
bool decode_fast_eligible(const DecodeParams &p, int wk);
int64_t decode_fast_slot_bytes(int kb, int vb, int Gv, int n_out, bool legacy);
// The legacy (per-token group) layouts the fast kernel takes: head_dim 128, 2 or 4
// bits, groups of 32 / 64 / 128 channels, fp16 scales and zeros.
bool decode_fast_legacy_shape(int D, int bits, int group_size, int meta_dtype);
// The fast kernel loads per-token meta rows of 1 or 2 groups in 16-byte pieces: with `heads`
// tiers of `rows_per_head` token rows each, every tier's meta must start on 16 bytes.
bool decode_fast_meta_aligned(int64_t rows_per_head, int Gv, int64_t heads);
int64_t decode_fast_lds_bytes(int64_t slot_bytes, int n_out);
int decode_fast_waves(int n_out);
hipError_t decode_fast_split_launch(const DecodeParams &p, int kb, int vb, int wk, hipStream_t s);
// Per-wave timeline of the fast kernel (timeline build only; 0 words / hipErrorNotSupported otherwise).
int64_t decode_fast_timeline_words();
hipError_t decode_fast_timeline_fetch(unsigned long long *host, int64_t words);
hipError_t decode_fast_timeline_clear(hipStream_t s);

}  // namespace akv
