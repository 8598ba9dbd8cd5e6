// Parameter blocks of the dequant, bitpack and importance kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace akv {

struct DequantParams {
    int kind;                     // AKV_WARM_AFFINE / AKV_WARM_LEGACY
    int nbh, Hkv, D;              // rows are (bh, token); nbh = B*Hkv (affine) or Hw (legacy)
    int64_t n_warm;
    int bits_k, bits_v;
    const void *kc, *vc;
    int kc_row, vc_row;
    const void *ks, *kz, *vs, *vz;
    int T, Gv;                    // affine
    int64_t nblk;
    int n_out;
    const int64_t *k_oidx, *v_oidx;
    const void *k_odata, *v_odata;
    int gs, lg, meta_dt, legacy_sym;  // legacy
    const int *sym_flags;
    int out_dt;
    void *k_out, *v_out;
    const int32_t *blk_of;        // affine: K-meta / outlier block of each token (else t / T)
    int64_t tok_stride;           // token rows per (bh) of codes, V meta, outlier values
    const int64_t *out_slot;      // output token row of each token (else the token's own row)
    int64_t out_tokens;           // output token rows per (bh) when out_slot is set
};

struct ImportanceParams {
    const void *attn;
    int attn_dt;
    int64_t B, H, M, N;
    float *scores;
    int64_t n_scores;
    float decay;
    int64_t m0;                   // first query row that counts (M - q_window, or 0)
    int pool;                     // average-pool width over keys (1 = none)
};

hipError_t dequant_launch(const DequantParams &p, hipStream_t s);
hipError_t stream_read_launch(const void *p, int64_t bytes, uint32_t *sink, hipStream_t s);
hipError_t bitpack_launch(const void *codes, void *packed, int64_t rows, int dim, int bits, int prow, hipStream_t s);
hipError_t bitunpack_launch(const void *packed, void *codes, int64_t rows, int prow, int dim, int bits, hipStream_t s);
hipError_t importance_launch(const ImportanceParams &p, hipStream_t s);
// bytes (a multiple of 16) of device memory at p set to zero by a kernel on s.
hipError_t zero_fill_launch(void *p, int64_t bytes, hipStream_t s);
// Demote selection: per row, the n smallest of `len` fp32 scores with positions [0, pf) and
// [max(0, len - pl), len) forced to +inf, ties to the lower index, indices ascending.
hipError_t select_launch(const float *scores, int64_t rows, int64_t len, int64_t n, int64_t pf, int64_t pl,
                         int64_t *out, hipStream_t s);

}  // namespace akv
