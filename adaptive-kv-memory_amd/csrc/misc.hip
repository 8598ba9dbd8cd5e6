// Dequant / unpack to dense values, device bit-packing, and the importance
// update from materialised attention weights.
#include "akv_common.h"
#include "misc.h"

namespace akv {

// ------------------------------------------------------------------ dequant
// One thread per (row, 8-channel chunk).  AFFINE: fp16 codes*scale + zero with
// two roundings, then outlier channels replaced (akv/affine_quantizer.py:112-124,
// :178-189).  LEGACY: fp32 u*s + z or (u - maxv//2)*s cast to the output dtype
// (akv/triton_ops.py:657-713, akv/fused_attention.py:281-317).
__global__ __launch_bounds__(256) void dequant_kernel(const DequantParams p) {
    const int nch = p.D / 8;
    const int64_t task = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t rows = (int64_t)p.nbh * p.n_warm;
    if (task >= rows * nch) return;
    const int64_t row = task / nch;  // (bh, token)
    const int ch8 = (int)(task % nch);
    const int64_t bh = row / p.n_warm, t = row % p.n_warm;
    for (int which = 0; which < 2; ++which) {
        void *out = which == 0 ? p.k_out : p.v_out;
        if (!out) continue;
        const int bits = which == 0 ? p.bits_k : p.bits_v;
        const unsigned char *codes = (const unsigned char *)(which == 0 ? p.kc : p.vc) + row * (which == 0 ? p.kc_row : p.vc_row);
        const void *sc = which == 0 ? p.ks : p.vs;
        const void *ze = which == 0 ? p.kz : p.vz;
        float vals[8];
        for (int i = 0; i < 8; ++i) {
            const int d = 8 * ch8 + i;
            const uint32_t c = extract_code(codes, d, bits);
            if (p.kind == AKV_WARM_AFFINE) {
                int64_t mi;
                if (which == 0) mi = (bh * p.nblk + t / p.T) * p.D + d;           // per channel, per block
                else mi = (bh * p.n_warm + t) * (p.D / p.Gv) + d / p.Gv;          // per token, per group
                const _Float16 s = ((const _Float16 *)sc)[mi], z = ((const _Float16 *)ze)[mi];
                _Float16 v = (_Float16)c * s;
                v = v + z;
                vals[i] = (float)v;
            } else {
                const int64_t mi = row * p.lg + d / p.gs;
                const float s = load_as_f32(sc, mi, p.meta_dt);
                const int sym = p.sym_flags ? p.sym_flags[which] : p.legacy_sym;
                float v;
                if (sym) v = ((float)c - (float)(((1 << bits) - 1) / 2)) * s;  // maxv // 2
                else {
                    v = (float)c * s;
                    v = v + load_as_f32(ze, mi, p.meta_dt);
                }
                vals[i] = v;
            }
        }
        if (p.kind == AKV_WARM_AFFINE && p.n_out > 0) {
            const int64_t *oi = (which == 0 ? p.k_oidx : p.v_oidx) + ((bh / p.Hkv) * p.nblk + t / p.T) * p.n_out;
            const _Float16 *od = (const _Float16 *)(which == 0 ? p.k_odata : p.v_odata) + row * p.n_out;
            for (int j = 0; j < p.n_out; ++j) {
                const int d = (int)oi[j];
                if (d / 8 == ch8) {
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        if (d % 8 == i) vals[i] = (float)od[j];
                }
            }
        }
        const int64_t o = row * p.D + 8 * ch8;
        for (int i = 0; i < 8; ++i) {
            if (p.out_dt == AKV_DT_F16) ((_Float16 *)out)[o + i] = (_Float16)vals[i];
            else if (p.out_dt == AKV_DT_BF16) ((uint16_t *)out)[o + i] = f32_to_bf16_rne(vals[i]);
            else ((float *)out)[o + i] = vals[i];
        }
    }
}

// ------------------------------------------------------------------ bitpack
// One thread per (row, group of 8 codes); bytes past the packed row are not written.
__global__ __launch_bounds__(256) void bitpack_kernel(const unsigned char *codes, unsigned char *packed, int64_t rows,
                                                      int dim, int bits, int prow) {
    const int ng = (dim + 7) / 8;
    const int64_t task = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (task >= rows * ng) return;
    const int64_t r = task / ng;
    const int g = (int)(task % ng);
    uint32_t c[8];
    for (int i = 0; i < 8; ++i) {
        const int d = 8 * g + i;
        c[i] = d < dim ? codes[r * dim + d] : 0u;
    }
    unsigned char out[8];
    int nb;
    if (bits == 4) {
        for (int i = 0; i < 4; ++i) out[i] = (unsigned char)(((c[2 * i] & 15u) << 4) | (c[2 * i + 1] & 15u));
        nb = 4;
    } else if (bits == 2) {
        for (int i = 0; i < 2; ++i)
            out[i] = (unsigned char)(((c[4 * i] & 3u) << 6) | ((c[4 * i + 1] & 3u) << 4) | ((c[4 * i + 2] & 3u) << 2) | (c[4 * i + 3] & 3u));
        nb = 2;
    } else {  // 3
        uint32_t W = 0;
        for (int i = 0; i < 8; ++i) W |= (c[i] & 7u) << (21 - 3 * i);
        out[0] = (unsigned char)(W >> 16);
        out[1] = (unsigned char)(W >> 8);
        out[2] = (unsigned char)W;
        nb = 3;
    }
    const int64_t base = (int64_t)g * nb;
    for (int i = 0; i < nb; ++i)
        if (base + i < prow) packed[r * prow + base + i] = out[i];
}

__global__ __launch_bounds__(256) void bitunpack_kernel(const unsigned char *packed, unsigned char *codes, int64_t rows,
                                                        int prow, int dim, int bits) {
    const int64_t task = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (task >= rows * dim) return;
    const int64_t r = task / dim;
    const int d = (int)(task % dim);
    codes[task] = (unsigned char)extract_code(packed + r * prow, d, bits);
}

// --------------------------------------------------------------- importance
// scores[n] = scores[n]*decay + sum_m (sum_{b,h} attn[b,h,m,n]) / (B*H)
__global__ __launch_bounds__(256) void importance_kernel(const ImportanceParams p) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n >= p.n_scores) return;
    float imp = 0.f;
    if (n < p.N) {
        const float inv_bh = (float)(p.B * p.H);
        for (int64_t m = 0; m < p.M; ++m) {
            float acc = 0.f;
            for (int64_t bh = 0; bh < p.B * p.H; ++bh)
                acc += load_as_f32(p.attn, (bh * p.M + m) * p.N + n, p.attn_dt);
            imp += acc / inv_bh;
        }
    }
    float s = p.scores[n] * p.decay;
    s = s + imp;
    p.scores[n] = s;
}

hipError_t dequant_launch(const DequantParams &p, hipStream_t s) {
    const int64_t tasks = (int64_t)p.nbh * p.n_warm * (p.D / 8);
    if (tasks == 0) return hipSuccess;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((tasks + 255) / 256)), dim3(256), 0, s, p);
    return hipGetLastError();
}
hipError_t bitpack_launch(const void *codes, void *packed, int64_t rows, int dim, int bits, int prow, hipStream_t s) {
    const int64_t tasks = rows * ((dim + 7) / 8);
    if (tasks == 0) return hipSuccess;
    hipLaunchKernelGGL(bitpack_kernel, dim3((unsigned)((tasks + 255) / 256)), dim3(256), 0, s,
                       (const unsigned char *)codes, (unsigned char *)packed, rows, dim, bits, prow);
    return hipGetLastError();
}
hipError_t bitunpack_launch(const void *packed, void *codes, int64_t rows, int prow, int dim, int bits, hipStream_t s) {
    const int64_t tasks = rows * dim;
    if (tasks == 0) return hipSuccess;
    hipLaunchKernelGGL(bitunpack_kernel, dim3((unsigned)((tasks + 255) / 256)), dim3(256), 0, s,
                       (const unsigned char *)packed, (unsigned char *)codes, rows, prow, dim, bits);
    return hipGetLastError();
}
hipError_t importance_launch(const ImportanceParams &p, hipStream_t s) {
    if (p.n_scores == 0) return hipSuccess;
    hipLaunchKernelGGL(importance_kernel, dim3((unsigned)((p.n_scores + 255) / 256)), dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace akv
