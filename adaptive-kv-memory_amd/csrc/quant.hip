// Gather -> block-affine quantize -> bit-pack (warm-tier demotion).
//
// Bit-exact restatement of AffineQuantizer.quantize_keys / quantize_values
// (akv/affine_quantizer.py:63-176) applied per T-token block (K, one scale and
// zero per channel) and per G-channel group of a token (V), followed by
// bitpack.pack (akv/bitpack.py:95-103); also the per-token-group evict
// quantizer of triton_kernels.fused_quantize_evict (akv/triton_kernels.py:464-500),
// which is the V rule applied to K as well.  Arithmetic is done the way the
// reference's CPU tensors do it: every op in fp32, rounded once to the input
// dtype (fp16 / bf16 / fp32), IEEE division, round-half-even, scale == 0
// gives NaN and NaN.to(uint8) == 0.
//
// One wave per (batch, head, block).  K lanes own a channel pair and walk the
// block's tokens (min/max is lane-local); codes are transposed through LDS
// and packed row by row.  V lanes own (token, group) and pack in registers.
#include "akv_common.h"
#include "quant.h"

namespace akv {

template <int DT>
__device__ __forceinline__ float rnd(float x) {
    if (DT == AKV_DT_F16) return (float)(_Float16)x;
    if (DT == AKV_DT_BF16) return bf16_to_f32(f32_to_bf16_rne(x));
    return x;
}
// input element i of a tensor of (runtime) dtype dt, as float
__device__ __forceinline__ float ld_in(const void *p, int64_t i, int dt) { return load_as_f32(p, i, dt); }
template <int DT>
__device__ __forceinline__ void st_meta(void *p, int64_t i, float v, int out_dt) {
    if (out_dt == AKV_DT_F16) ((_Float16 *)p)[i] = (_Float16)v;
    else if (out_dt == AKV_DT_BF16) ((uint16_t *)p)[i] = f32_to_bf16_rne(v);
    else ((float *)p)[i] = v;
}

// scale/zero of one quantization group from its min / max (input-dtype arithmetic)
template <int DT>
__device__ __forceinline__ void scale_zero(float mn, float mx, int maxv, float lo, float &scale, float &zero) {
    float s = rnd<DT>(mx - mn);
    s = rnd<DT>(s / (float)maxv);
    if (!(s != s)) s = fmaxf(s, lo);  // clamp(min=1e-8) as the dtype sees 1e-8; NaN stays
    scale = s;
    zero = mn;
}
template <int DT>
__device__ __forceinline__ uint32_t quant_code(float x, float zero, float scale, int maxv) {
    float q = rnd<DT>(x - zero);
    q = rnd<DT>(q / scale);
    q = rintf(q);
    if (q != q) return 0u;             // NaN -> 0
    q = fminf(fmaxf(q, 0.0f), (float)maxv);
    return (uint32_t)q;
}

// Append the bitpack bytes of 8 codes (c[0..7]) to a little-endian dword stream.
struct ByteStream {
    uint32_t w[32];
    int nb;
    __device__ __forceinline__ void put(uint32_t byte) {
        const int i = nb >> 2, s = (nb & 3) * 8;
        if (s == 0) w[i] = byte;
        else w[i] |= byte << s;
        ++nb;
    }
};
__device__ __forceinline__ void pack8(ByteStream &bs, const uint32_t *c, int bits) {
    if (bits == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) bs.put(((c[2 * i] & 15u) << 4) | (c[2 * i + 1] & 15u));
    } else if (bits == 2) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            bs.put(((c[4 * i] & 3u) << 6) | ((c[4 * i + 1] & 3u) << 4) | ((c[4 * i + 2] & 3u) << 2) | (c[4 * i + 3] & 3u));
    } else if (bits == 3) {
        uint32_t W = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) W |= (c[i] & 7u) << (21 - 3 * i);
        bs.put((W >> 16) & 0xFFu);
        bs.put((W >> 8) & 0xFFu);
        bs.put(W & 0xFFu);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) bs.put(c[i] & 0xFFu);
    }
}

// per-(batch, block) outlier channels: rank by mean over heads of the L2 norm
// over the block's tokens (akv/affine_quantizer.py:76-80), ties -> lower index.
template <int DT>
__global__ __launch_bounds__(256) void outlier_select_kernel(const QuantParams p) {
    __shared__ float cn[2][256];
    const int blk = blockIdx.x, b = blockIdx.y;
    const int64_t t0 = (int64_t)blk * p.T, t1 = min(t0 + p.T, p.n_sel);
    for (int which = 0; which < 2; ++which) {
        const void *x = which == 0 ? p.k : p.v;
        if (!x) continue;
        for (int d = threadIdx.x; d < p.D; d += 256) {
            float acc = 0.f;
            for (int h = 0; h < p.H; ++h) {
                float ss = 0.f;
                for (int64_t t = t0; t < t1; ++t) {
                    const int64_t src = p.sel ? min(max(p.sel[(int64_t)b * p.n_sel + t], (int64_t)0), p.n_src - 1) : t;
                    const float v = ld_in(x, (((int64_t)b * p.H + h) * p.n_src + src) * p.D + d, p.in_dt);
                    ss += v * v;
                }
                acc += sqrtf(ss);
            }
            cn[which][d] = acc / (float)p.H;
        }
    }
    __syncthreads();
    if (threadIdx.x < 2) {
        const int which = threadIdx.x;
        const void *x = which == 0 ? p.k : p.v;
        int64_t *oidx = which == 0 ? p.k_oidx : p.v_oidx;
        if (x && oidx) {
            uint32_t taken[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int j = 0; j < p.n_out; ++j) {
                int best = -1;
                float bv = 0.f;
                for (int d = 0; d < p.D; ++d) {
                    if (taken[d >> 5] & (1u << (d & 31))) continue;
                    const float v = cn[which][d];
                    if (best < 0 || v > bv) { best = d; bv = v; }
                }
                taken[best >> 5] |= 1u << (best & 31);
                oidx[((int64_t)b * p.nblk + blk) * p.n_out + j] = best;
            }
        }
    }
}

template <int DT>
__device__ __forceinline__ bool is_outlier(const int64_t *oidx, int n_out, int d, int *slot) {
    for (int j = 0; j < n_out; ++j)
        if ((int)oidx[j] == d) { *slot = j; return true; }
    return false;
}

template <int DT>
__global__ __launch_bounds__(256) void quant_kernel(const QuantParams p) {
    __shared__ __align__(16) unsigned char codes_lds[4][32 * 128];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t blk = (int64_t)blockIdx.x * 4 + wave;
    const int h = blockIdx.y, b = blockIdx.z;
    if (blk >= p.nblk) return;
    const int64_t t0 = blk * p.T, t1 = min(t0 + p.T, p.n_sel);
    const int64_t bh = (int64_t)b * p.H + h;
    const float lo = p.lo;
    unsigned char *clds = codes_lds[wave];

    // ------------------------------------------------------------------ K
    if (p.k && p.k_mode == 0) {
        const int maxv = (1 << p.bits_k) - 1;
        const int64_t *oidx = p.n_out ? p.k_oidx + ((int64_t)b * p.nblk + blk) * p.n_out : nullptr;
        const int npl = p.D / 64;  // channels per lane: 2 (D=128) or 1 (D=64)
        float mn[2] = {INFINITY, INFINITY}, mx[2] = {-INFINITY, -INFINITY};
        int oslot[2] = {-1, -1};
        for (int c = 0; c < npl; ++c) {
            int sl;
            if (oidx && is_outlier<DT>(oidx, p.n_out, npl * lane + c, &sl)) oslot[c] = sl;
        }
        for (int64_t t = t0; t < t1; ++t) {
            const int64_t src = p.sel ? min(max(p.sel[(int64_t)b * p.n_sel + t], (int64_t)0), p.n_src - 1) : t;
            for (int c = 0; c < npl; ++c) {
                float x = ld_in(p.k, (bh * p.n_src + src) * p.D + npl * lane + c, p.in_dt);
                if (oslot[c] >= 0) x = 0.f;
                mn[c] = fminf(mn[c], x);
                mx[c] = fmaxf(mx[c], x);
            }
        }
        float sc[2], ze[2];
        for (int c = 0; c < npl; ++c) {
            scale_zero<DT>(mn[c], mx[c], maxv, lo, sc[c], ze[c]);
            const int64_t mi = (bh * p.nblk + blk) * p.D + npl * lane + c;
            ((_Float16 *)p.k_scale)[mi] = (_Float16)sc[c];
            ((_Float16 *)p.k_zero)[mi] = (_Float16)ze[c];
        }
        // quantize in sub-blocks of 32 tokens, transposed through LDS, packed per row
        const int rowb = p.k_row;             // packed bytes per token row
        const int segb = 32 * p.bits_k / 8;  // packed bytes per 32 channels
        for (int64_t s0 = t0; s0 < t1; s0 += 32) {
            const int64_t s1 = min(s0 + 32, t1);
            for (int64_t t = s0; t < s1; ++t) {
                const int64_t src = p.sel ? min(max(p.sel[(int64_t)b * p.n_sel + t], (int64_t)0), p.n_src - 1) : t;
                for (int c = 0; c < npl; ++c) {
                    float x = ld_in(p.k, (bh * p.n_src + src) * p.D + npl * lane + c, p.in_dt);
                    if (oslot[c] >= 0) {
                        ((_Float16 *)p.k_odata)[(bh * p.n_sel + t) * p.n_out + oslot[c]] = (_Float16)x;
                        x = 0.f;
                    }
                    clds[(t - s0) * 128 + npl * lane + c] = (unsigned char)quant_code<DT>(x, ze[c], sc[c], maxv);
                }
            }
            __builtin_amdgcn_wave_barrier();
            const int nseg = p.D / 32;
            const int ntask = (int)(s1 - s0) * nseg;
            for (int task = lane; task < ntask; task += 64) {
                const int tt = task / nseg, sg = task % nseg;
                ByteStream bs;
                bs.nb = 0;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    uint32_t c8[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) c8[i] = clds[tt * 128 + 32 * sg + 8 * q + i];
                    pack8(bs, c8, p.bits_k);
                }
                unsigned char *dst = (unsigned char *)p.k_codes + (bh * p.n_sel + s0 + tt) * rowb + segb * sg;
                for (int q = 0; q < segb / 4; ++q) ((uint32_t *)dst)[q] = bs.w[q];
            }
            __builtin_amdgcn_wave_barrier();
        }
    }

    // ----------------------------------------------- V (and K in group mode)
    for (int which = 0; which < 2; ++which) {
        const void *x = which == 0 ? p.k : p.v;
        if (!x || (which == 0 && p.k_mode == 0)) continue;
        const int bits = which == 0 ? p.bits_k : p.bits_v;
        const int sbits = which == 0 ? p.sbits_k : p.sbits_v;  // storage bits (8 = raw codes)
        const int maxv = (1 << bits) - 1;
        const int G = which == 0 ? p.G_k : p.G_v;
        const int pD = p.pD;
        const int ng = pD / G;
        const int rowb = which == 0 ? p.k_row : p.v_row;
        const int grpb = G * sbits / 8;
        void *codes = which == 0 ? p.k_codes : p.v_codes;
        void *msc = which == 0 ? p.k_scale : p.v_scale;
        void *mze = which == 0 ? p.k_zero : p.v_zero;
        const int64_t *oidx =
            (p.n_out && which == 1) ? p.v_oidx + ((int64_t)b * p.nblk + blk) * p.n_out : nullptr;
        _Float16 *odata = which == 1 ? (_Float16 *)p.v_odata : nullptr;
        const int ntask = (int)(t1 - t0) * ng;
        for (int task = lane; task < ntask; task += 64) {
            const int64_t t = t0 + task / ng;
            const int g = task % ng;
            const int64_t src = p.sel ? min(max(p.sel[(int64_t)b * p.n_sel + t], (int64_t)0), p.n_src - 1) : t;
            const int64_t rowi = (bh * p.n_src + src) * p.D;
            float mn = INFINITY, mx = -INFINITY;
            for (int c = 0; c < G; ++c) {
                const int d = g * G + c;
                float xv = d < p.D ? ld_in(x, rowi + d, p.in_dt) : 0.f;  // channels past D: zero padding
                int sl;
                if (oidx && d < p.D && is_outlier<DT>(oidx, p.n_out, d, &sl)) {
                    odata[(bh * p.n_sel + t) * p.n_out + sl] = (_Float16)xv;
                    xv = 0.f;
                }
                mn = fminf(mn, xv);
                mx = fmaxf(mx, xv);
            }
            float sc, ze;
            if (p.symmetric) {  // akv/quantizer.py:113-119
                const float absmax = fmaxf(fabsf(mn), fabsf(mx));
                sc = absmax / ((float)maxv / 2.0f);
                sc = fmaxf(sc, lo);
                ze = 0.0f;
            } else {
                scale_zero<DT>(mn, mx, maxv, lo, sc, ze);
            }
            const int64_t mi = (bh * p.n_sel + t) * ng + g;
            st_meta<DT>(msc, mi, sc, p.meta_dt);
            st_meta<DT>(mze, mi, ze, p.meta_dt);
            ByteStream bs;
            bs.nb = 0;
            for (int c0 = 0; c0 < G; c0 += 8) {
                uint32_t c8[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int d = g * G + c0 + i;
                    float xv = d < p.D ? ld_in(x, rowi + d, p.in_dt) : 0.f;
                    int sl;
                    if (oidx && d < p.D && is_outlier<DT>(oidx, p.n_out, d, &sl)) xv = 0.f;
                    if (p.symmetric) {  // round(x/s).clamp(-maxv//2, maxv//2) + maxv//2, uint8 wrap
                        float q = rintf(xv / sc);
                        q = fminf(fmaxf(q, (float)(-((maxv + 1) / 2))), (float)(maxv / 2));
                        c8[i] = (uint32_t)((int)q + maxv / 2) & 0xFFu;
                    } else {
                        c8[i] = quant_code<DT>(xv, ze, sc, maxv);
                    }
                }
                pack8(bs, c8, sbits);
            }
            unsigned char *dst = (unsigned char *)codes + (bh * p.n_sel + t) * rowb + (int64_t)grpb * g;
            for (int q = 0; q < grpb / 4; ++q) ((uint32_t *)dst)[q] = bs.w[q];
        }
    }
}

hipError_t quant_launch(const QuantParams &p, hipStream_t s) {
    hipError_t e;
    if (p.n_out > 0) {
        dim3 g((unsigned)p.nblk, p.B);
        hipLaunchKernelGGL(outlier_select_kernel<AKV_DT_F32>, g, dim3(256), 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    dim3 grid((unsigned)((p.nblk + 3) / 4), p.H, p.B);
    if (p.ar_dt == AKV_DT_F16) hipLaunchKernelGGL(quant_kernel<AKV_DT_F16>, grid, dim3(256), 0, s, p);
    else if (p.ar_dt == AKV_DT_BF16) hipLaunchKernelGGL(quant_kernel<AKV_DT_BF16>, grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(quant_kernel<AKV_DT_F32>, grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace akv
