// Host/device parameter block of the chunked-prefill attention kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace akv {

struct PrefillParams {
    int B, Hq, Hkv, M, g, R;        // R = g * M query rows per (batch, kv-head)
    int q_bf16;                     // q and out are bf16 (else fp16)
    const void *q;                  // [B][Hq][M][128]
    void *out;                      // [B][Hq][M][128]
    const _Float16 *khot, *vhot;    // [B][Hkv][n_hot][128]
    int64_t n_hot;
    const void *kc, *vc;            // block-affine warm tier, D = 128
    const _Float16 *ks, *kz, *vs, *vz;
    int64_t n_warm, nblk;
    int T, Gv, bits_k, bits_v;
    float scale_log2;               // sm_scale * log2(e)
    int n_row_tiles;                // ceil(R / rows per workgroup)
    int nsplit;                     // token splits (partials merged by decode_reduce_kernel)
    int64_t tiles_per_split;        // 32-token tiles per split (hot tiles first, then warm)
    float *part;                    // partials, decode layout (16-row chunks), when nsplit > 1
    int nchunk, prows;              // 16-row chunks of R and rows per partial (decode layout)
    const void *kcur, *vcur;        // the chunk's own K / V [B][Hkv][M][128] in q's dtype (or null):
    int n_cur;                      // attended causally after the cache; n_cur = M (0 without them)
};

constexpr int kPrefillRows = 256;   // query rows per workgroup

// Launch the split kernel and, when nsplit > 1, the merge.
hipError_t prefill_launch(const PrefillParams &p, hipStream_t s);

}  // namespace akv
