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

// ---------------------------------------------------------------- fast path
// fp16 input and arithmetic, D = 128, K per channel over 32-token blocks, V per
// token over G-channel groups, no outliers: one wave per (batch, head, block).
// Lane (cg = lane % 16, tg = lane / 16) holds channels 8cg .. 8cg+7 of the
// block's tokens 8tg .. 8tg+7 (one 16-byte load per token and tensor).
//   min / max: packed fp16 min / max in the lane, then across the lanes that
//   share a channel (K: the 4 token groups) or a group (V: G/8 channel groups);
//   scale = round16(round16(max - min) * (1/maxv)) -- equal to the reference's
//   division by maxv for every fp16 value, checked exhaustively;
//   code = clamp(rint(round16(round16(x - zero) / scale)), 0, maxv) computed as
//   one fused multiply by r = 1/scale (fp32, correctly rounded) rounded once
//   to fp16 (v_fma_mix), then + 1024 (fp16 rounding to an integer, ties to
//   even) and a clamp in [1024, 1024 + maxv]: the same codes as the
//   reference for every fp16 quotient, checked exhaustively over all fp16
//   (x - zero, scale) pairs; NaN gives 0 and +inf gives maxv as there.
// Packed rows go through LDS and leave as one contiguous 16-byte-per-lane
// store per tensor (a block's rows are contiguous in the packed layout).

namespace {

// fp16 of a * r (r fp32) with one rounding, for the low / high half of a.
__device__ __forceinline__ uint32_t mul_mix2(uint32_t a, float r_lo, float r_hi) {
    uint32_t d = 0;
    asm volatile("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "+v"(d) : "v"(a), "v"(r_lo));
    asm volatile("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(d) : "v"(a), "v"(r_hi));
    return d;
}

// codes of a pair of quotients d (fp16x2): (1024 + code) in each half
__device__ __forceinline__ uint32_t code2(uint32_t d, h2 hi_clamp) {
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    h2 u = as_h2(d) + k1024;
    u = __builtin_elementwise_max(u, k1024);
    u = __builtin_elementwise_min(u, hi_clamp);
    return as_u32(u);
}

__device__ __forceinline__ h2 hmin2(h2 a, h2 b) { return __builtin_elementwise_min(a, b); }
__device__ __forceinline__ h2 hmax2(h2 a, h2 b) { return __builtin_elementwise_max(a, b); }

// scale of a (min, max) pair held as fp16: round16(round16(mx - mn) * (1/maxv))
__device__ __forceinline__ float scale_of(_Float16 mn, _Float16 mx, float inv_maxv) {
    const _Float16 d = mx - mn;
    return (float)(_Float16)((float)d * inv_maxv);
}

// packed bytes of 8 codes (held as 1024 + code in the fp16 halves of c[0..3])
template <int BITS>
__device__ __forceinline__ void pack_row(const uint32_t *c, unsigned char *dst) {
    uint32_t v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = c[i] & 0x3FFu;
        v[2 * i + 1] = (c[i] >> 16) & 0x3FFu;
    }
    if (BITS == 4) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) w |= ((v[2 * i] << 4) | v[2 * i + 1]) << (8 * i);
        *(uint32_t *)dst = w;
    } else if (BITS == 2) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) w |= ((v[4 * i] << 6) | (v[4 * i + 1] << 4) | (v[4 * i + 2] << 2) | v[4 * i + 3]) << (8 * i);
        *(uint16_t *)dst = (uint16_t)w;
    } else {
        uint32_t W = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) W |= v[i] << (21 - 3 * i);
        dst[0] = (unsigned char)(W >> 16);
        dst[1] = (unsigned char)(W >> 8);
        dst[2] = (unsigned char)W;
    }
}

template <int N>
__device__ __forceinline__ uint32_t xor_lane(uint32_t x) { return (uint32_t)__shfl_xor((int)x, N); }

}  // namespace

// codes and K meta leave with non-temporal stores (written once; measured ~3%
// faster at the 64k demotion than write-back stores)
#define QSTORE(v, ptr) __builtin_nontemporal_store((v), (ptr))
template <int BK, int BV, int NG>
__global__ __launch_bounds__(256) void quant_fast_kernel(const QuantParams p) {
    constexpr int KR = 16 * BK, VR = 16 * BV, LG = 16 / NG;  // lanes (channel groups of 8) per V group
    __shared__ __align__(16) unsigned char stage[4][2][32 * 64 + 2 * 32 * 4 * 2];  // codes, then V meta
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t blk = (int64_t)blockIdx.x * 4 + wave;
    const int h = blockIdx.y, b = blockIdx.z;
    if (blk >= p.nblk) return;
    const int cg = lane & 15, tg = lane >> 4;
    const int64_t t0 = blk * 32;
    const int nv = (int)min((int64_t)32, p.n_sel - t0);  // valid tokens of the block
    const int64_t bh = (int64_t)b * p.H + h;

    // ---- loads: tokens 8tg + i (invalid ones repeat token t0: min / max unchanged)
    u4 kx[8], vx[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int tl = 8 * tg + i;
        const int64_t t = t0 + (tl < nv ? tl : 0);
        const int64_t src = p.sel ? min(max(p.sel[(int64_t)b * p.n_sel + t], (int64_t)0), p.n_src - 1) : t;
        const int64_t off = (bh * p.n_src + src) * 128 + 8 * cg;
        // non-temporal: each row is read once (measured ~2% faster at the 64k demotion)
        if (p.k) kx[i] = __builtin_nontemporal_load((const u4 *)((const _Float16 *)p.k + off));
        if (p.v) vx[i] = __builtin_nontemporal_load((const u4 *)((const _Float16 *)p.v + off));
    }

    // ---------------------------------------------------------------- K
    if (p.k) {
        constexpr int MAXV = (1 << BK) - 1;
        const float inv = 1.0f / (float)MAXV;
        h2 mn[4], mx[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) mn[j] = mx[j] = as_h2(kx[0][j]);
#pragma unroll
        for (int i = 1; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                mn[j] = hmin2(mn[j], as_h2(kx[i][j]));
                mx[j] = hmax2(mx[j], as_h2(kx[i][j]));
            }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            mn[j] = hmin2(mn[j], as_h2(xor_lane<16>(as_u32(mn[j]))));
            mx[j] = hmax2(mx[j], as_h2(xor_lane<16>(as_u32(mx[j]))));
            mn[j] = hmin2(mn[j], as_h2(xor_lane<32>(as_u32(mn[j]))));
            mx[j] = hmax2(mx[j], as_h2(xor_lane<32>(as_u32(mx[j]))));
        }
        float r[8];
        uint32_t sc[4], nz[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float s0 = scale_of(mn[j][0], mx[j][0], inv), s1 = scale_of(mn[j][1], mx[j][1], inv);
            r[2 * j] = 1.0f / s0;
            r[2 * j + 1] = 1.0f / s1;
            sc[j] = as_u32((h2){(_Float16)s0, (_Float16)s1});
            nz[j] = as_u32(mn[j]) ^ 0x80008000u;  // -zero
        }
        if (tg == 0) {
            const int64_t mi = (bh * p.nblk + blk) * 128 + 8 * cg;
            QSTORE(((u4){sc[0], sc[1], sc[2], sc[3]}), (u4 *)((_Float16 *)p.k_scale + mi));
            QSTORE(((u4){as_u32(mn[0]), as_u32(mn[1]), as_u32(mn[2]), as_u32(mn[3])}), (u4 *)((_Float16 *)p.k_zero + mi));
        }
        const h2 hic = {(_Float16)(1024.0f + MAXV), (_Float16)(1024.0f + MAXV)};
        unsigned char *st = stage[wave][0];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t c[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t q = as_u32(as_h2(kx[i][j]) + as_h2(nz[j]));
                c[j] = code2(mul_mix2(q, r[2 * j], r[2 * j + 1]), hic);
            }
            pack_row<BK>(c, st + (8 * tg + i) * KR + cg * BK);
        }
        __builtin_amdgcn_wave_barrier();
        const int nbytes = nv * KR;
        unsigned char *dst = (unsigned char *)p.k_codes + (bh * p.n_sel + t0) * KR;
        for (int o = 16 * lane; o < nbytes; o += 1024) QSTORE(*(const u4 *)(st + o), (u4 *)(dst + o));
    }

    // ---------------------------------------------------------------- V
    if (p.v) {
        constexpr int MAXV = (1 << BV) - 1;
        const float inv = 1.0f / (float)MAXV;
        // per token: min / max over the lane's 8 channels, packed two tokens per h2
        h2 mn2[4], mx2[4];
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
            _Float16 lo_mn, lo_mx, hi_mn, hi_mx;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const u4 x = vx[2 * i2 + e];
                h2 a = hmin2(hmin2(as_h2(x[0]), as_h2(x[1])), hmin2(as_h2(x[2]), as_h2(x[3])));
                h2 c = hmax2(hmax2(as_h2(x[0]), as_h2(x[1])), hmax2(as_h2(x[2]), as_h2(x[3])));
                const _Float16 m0 = __builtin_fminf16(a[0], a[1]), m1 = __builtin_fmaxf16(c[0], c[1]);
                if (e == 0) { lo_mn = m0; lo_mx = m1; } else { hi_mn = m0; hi_mx = m1; }
            }
            mn2[i2] = (h2){lo_mn, hi_mn};
            mx2[i2] = (h2){lo_mx, hi_mx};
        }
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
            if (LG >= 2) {
                mn2[i2] = hmin2(mn2[i2], as_h2(xor_lane<1>(as_u32(mn2[i2]))));
                mx2[i2] = hmax2(mx2[i2], as_h2(xor_lane<1>(as_u32(mx2[i2]))));
            }
            if (LG >= 4) {
                mn2[i2] = hmin2(mn2[i2], as_h2(xor_lane<2>(as_u32(mn2[i2]))));
                mx2[i2] = hmax2(mx2[i2], as_h2(xor_lane<2>(as_u32(mx2[i2]))));
            }
            if (LG >= 8) {
                mn2[i2] = hmin2(mn2[i2], as_h2(xor_lane<4>(as_u32(mn2[i2]))));
                mx2[i2] = hmax2(mx2[i2], as_h2(xor_lane<4>(as_u32(mx2[i2]))));
            }
            if (LG >= 16) {
                mn2[i2] = hmin2(mn2[i2], as_h2(xor_lane<8>(as_u32(mn2[i2]))));
                mx2[i2] = hmax2(mx2[i2], as_h2(xor_lane<8>(as_u32(mx2[i2]))));
            }
        }
        const int gv = cg / LG;
        unsigned char *st = stage[wave][1];
        unsigned char *mst = st + 32 * 64;  // [token][group] scale then zero, fp16
        const h2 hic = {(_Float16)(1024.0f + MAXV), (_Float16)(1024.0f + MAXV)};
#pragma unroll
        for (int i2 = 0; i2 < 4; ++i2) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int i = 2 * i2 + e, tl = 8 * tg + i;
                const _Float16 zmn = mn2[i2][e];
                const float s = scale_of(zmn, mx2[i2][e], inv);
                const float r = 1.0f / s;
                if (cg % LG == 0) {
                    ((_Float16 *)mst)[tl * NG + gv] = (_Float16)s;
                    ((_Float16 *)mst)[32 * NG + tl * NG + gv] = zmn;
                }
                const h2 nzz = {(_Float16)(-zmn), (_Float16)(-zmn)};
                uint32_t c[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t q = as_u32(as_h2(vx[i][j]) + nzz);
                    c[j] = code2(mul_mix2(q, r, r), hic);
                }
                pack_row<BV>(c, st + tl * VR + cg * BV);
            }
        }
        __builtin_amdgcn_wave_barrier();
        const int nbytes = nv * VR;
        unsigned char *dst = (unsigned char *)p.v_codes + (bh * p.n_sel + t0) * VR;
        for (int o = 16 * lane; o < nbytes; o += 1024) QSTORE(*(const u4 *)(st + o), (u4 *)(dst + o));
        // meta: nv tokens x NG fp16 scales, then zeros (contiguous per block)
        const int mh = nv * NG;
        _Float16 *ds = (_Float16 *)p.v_scale + (bh * p.n_sel + t0) * NG;
        _Float16 *dz = (_Float16 *)p.v_zero + (bh * p.n_sel + t0) * NG;
        for (int o = lane; o < mh; o += 64) {
            ds[o] = ((const _Float16 *)mst)[o];
            dz[o] = ((const _Float16 *)mst)[32 * NG + o];
        }
    }
}

static bool quant_fast_eligible(const QuantParams &p) {
    const bool al = (((uintptr_t)p.k | (uintptr_t)p.v | (uintptr_t)p.k_codes | (uintptr_t)p.v_codes |
                      (uintptr_t)p.k_scale | (uintptr_t)p.k_zero) & 15u) == 0;
    return al && p.in_dt == AKV_DT_F16 && p.ar_dt == AKV_DT_F16 && p.D == 128 && p.pD == 128 && p.T == 32 &&
           p.k_mode == 0 && p.n_out == 0 && !p.symmetric && p.meta_dt == AKV_DT_F16 &&
           p.bits_k >= 2 && p.bits_k <= 4 && p.bits_v >= 2 && p.bits_v <= 4 &&
           p.sbits_k == p.bits_k && p.sbits_v == p.bits_v && (p.G_v == 32 || p.G_v == 64 || p.G_v == 128);
}

template <int BK, int BV>
static void launch_quant_fast(const QuantParams &p, dim3 grid, hipStream_t s) {
    if (p.G_v == 32) hipLaunchKernelGGL((quant_fast_kernel<BK, BV, 4>), grid, dim3(256), 0, s, p);
    else if (p.G_v == 64) hipLaunchKernelGGL((quant_fast_kernel<BK, BV, 2>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((quant_fast_kernel<BK, BV, 1>), grid, dim3(256), 0, s, p);
}

hipError_t quant_launch(const QuantParams &p, hipStream_t s) {
    hipError_t e;
    if (p.n_out > 0) {
        dim3 g((unsigned)p.nblk, p.B);
        hipLaunchKernelGGL(outlier_select_kernel<AKV_DT_F32>, g, dim3(256), 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    dim3 grid((unsigned)((p.nblk + 3) / 4), p.H, p.B);
    if (quant_fast_eligible(p)) {
#define AKV_QKV(a, c) \
    if (p.bits_k == a && p.bits_v == c) launch_quant_fast<a, c>(p, grid, s);
        AKV_QKV(2, 2) AKV_QKV(2, 3) AKV_QKV(2, 4) AKV_QKV(3, 2) AKV_QKV(3, 3) AKV_QKV(3, 4) AKV_QKV(4, 2)
        AKV_QKV(4, 3) AKV_QKV(4, 4)
#undef AKV_QKV
        return hipGetLastError();
    }
    if (p.ar_dt == AKV_DT_F16) hipLaunchKernelGGL(quant_kernel<AKV_DT_F16>, grid, dim3(256), 0, s, p);
    else if (p.ar_dt == AKV_DT_BF16) hipLaunchKernelGGL(quant_kernel<AKV_DT_BF16>, grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(quant_kernel<AKV_DT_F32>, grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace akv
