// Parameter block of the quantize + pack kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace akv {

struct QuantParams {
    int B, H, D, pD;             // pD: D rounded up to the group size (evict padding)
    int in_dt;                   // AKV_DT_* of k / v (loads)
    int ar_dt;                   // AKV_DT_* the arithmetic is rounded to
    float lo;                    // scale clamp(min=...) as the arithmetic dtype sees it
    int symmetric;               // KVQuantizer symmetric branch
    const void *k, *v;           // [B][H][n_src][D]
    int64_t n_src, n_sel;
    const int64_t *sel;          // [B][n_sel] or null
    int bits_k, bits_v;          // quantization widths
    int sbits_k, sbits_v;        // storage widths (8 = one byte per code)
    int T;                       // K token block (k_mode 0) / work block
    int G_k, G_v;                // channel groups (K in group mode, V)
    int64_t nblk;
    int n_out;
    int k_mode;                  // 0: per-channel over T-token blocks, 1: per-token groups
    int meta_dt;                 // dtype of written scales / zeros
    int k_row, v_row;            // packed bytes per token row
    void *k_codes, *k_scale, *k_zero;
    void *v_codes, *v_scale, *v_zero;
    int64_t *k_oidx, *v_oidx;
    void *k_odata, *v_odata;
};

hipError_t quant_launch(const QuantParams &p, hipStream_t s);

}  // namespace akv
