// Dequant / unpack to dense values, device bit-packing, and the importance
// update from materialised attention weights.
#include <atomic>

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
    const int ch8 = (int)(task % nch);
    const int64_t bh = task / nch / p.n_warm, t = task / nch % p.n_warm;
    const int64_t row = bh * p.tok_stride + t;  // input row (bh, token)
    const int64_t blk = p.blk_of ? (int64_t)p.blk_of[t] : t / p.T;
    const int64_t orow = p.out_slot ? bh * p.out_tokens + p.out_slot[t] : bh * p.n_warm + t;
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
                if (which == 0) mi = (bh * p.nblk + blk) * p.D + d;              // per channel, per block
                else mi = row * (p.D / p.Gv) + d / p.Gv;                          // per token, per group
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
            const int64_t *oi = (which == 0 ? p.k_oidx : p.v_oidx) + ((bh / p.Hkv) * p.nblk + blk) * p.n_out;
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
        const int64_t o = orow * p.D + 8 * ch8;
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
// scores[n] = scores[n]*decay + imp[n], imp[n] = sum_{m >= m0} (sum_{b,h} attn[b,h,m,n]) / (B*H);
// with pool > 1 imp is first average-pooled over keys: (1/pool) sum_{j<pool} imp[n - pool/2 + j]
// (zero outside [0, N)).  A workgroup owns 256 keys; with pooling it also sums the
// pool - 1 keys of its halo into LDS, so each attention element is read about once.
constexpr int kImpTile = 256, kImpMaxPool = 64;
__device__ __forceinline__ float key_importance(const ImportanceParams &p, int64_t n) {
    if (n < 0 || n >= p.N) return 0.f;
    const float inv_bh = (float)(p.B * p.H);
    float imp = 0.f;
    for (int64_t m = p.m0; m < p.M; ++m) {
        float acc = 0.f;
        for (int64_t bh = 0; bh < p.B * p.H; ++bh) acc += load_as_f32(p.attn, (bh * p.M + m) * p.N + n, p.attn_dt);
        imp += acc / inv_bh;
    }
    return imp;
}
__global__ __launch_bounds__(kImpTile) void importance_kernel(const ImportanceParams p) {
    __shared__ float halo[kImpTile + kImpMaxPool];
    const int64_t n0 = (int64_t)blockIdx.x * kImpTile, n = n0 + threadIdx.x;
    float imp;
    if (p.pool > 1) {
        const int pad = p.pool / 2, width = kImpTile + p.pool - 1;
        for (int i = threadIdx.x; i < width; i += kImpTile) halo[i] = key_importance(p, n0 - pad + i);
        __syncthreads();
        imp = 0.f;
        for (int j = 0; j < p.pool; ++j) imp += halo[threadIdx.x + j];
        imp = imp / (float)p.pool;
        if (n >= p.N) imp = 0.f;  // pooled output is trimmed to the N keys
    } else {
        imp = key_importance(p, n);
    }
    if (n >= p.n_scores) return;
    float s = p.scores[n] * p.decay;
    s = s + imp;
    p.scores[n] = s;
}

// Without key pooling: a workgroup owns 64 keys and its RG waves split the (batch x
// head) rows into RG contiguous ranges, 8 loads in flight per lane.  The row loads of
// a wave cover 64 consecutive keys (256 coalesced bytes at fp32).  Sum order, per
// query row m >= m0: over the rows of a range, then over the ranges in range order,
// then divided by B*H; the per-query means are then added in query order -- the
// reference's association (mean over batch and heads, then the sum over queries),
// with the (batch, head) sum itself in another order than torch's reduction (fp32
// rounding may differ in the last bits).  RG = 16 when there are too few key tiles to
// fill the GPU with RG = 4.
constexpr int kImpKeys = 64;
template <int RG>
__global__ __launch_bounds__(64 * RG) void importance_rows_kernel(const ImportanceParams p) {
    __shared__ float part[RG][kImpKeys];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t n = (int64_t)blockIdx.x * kImpKeys + lane;
    const int64_t bhn = p.B * p.H, per = (bhn + RG - 1) / RG;
    const int64_t bh0 = min(bhn, per * w), bh1 = min(bhn, bh0 + per);
    float imp = 0.f;  // wave 0: the sum over queries of the per-query means
    for (int64_t m = p.m0; m < p.M; ++m) {
        float acc = 0.f;
        if (n < p.N) {
            int64_t bh = bh0;
            for (; bh + 8 <= bh1; bh += 8) {
                float x[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = load_as_f32(p.attn, ((bh + j) * p.M + m) * p.N + n, p.attn_dt);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc += x[j];
            }
            for (; bh < bh1; ++bh) acc += load_as_f32(p.attn, (bh * p.M + m) * p.N + n, p.attn_dt);
        }
        part[w][lane] = acc;
        __syncthreads();
        if (w == 0) {
            float tot = 0.f;
#pragma unroll
            for (int r = 0; r < RG; ++r) tot += part[r][lane];
            imp += tot / (float)bhn;
        }
        __syncthreads();  // part is rewritten for the next query row
    }
    if (w != 0 || n >= p.n_scores) return;
    if (n >= p.N) imp = 0.f;
    float sc = p.scores[n] * p.decay;
    sc = sc + imp;
    p.scores[n] = sc;
}

// ------------------------------------------------------------ demote selection
// One workgroup (1024 threads) per row.  Scores become order-preserving 32-bit
// keys (-0 as +0, NaN above +inf, protected positions = +inf); a 4-pass radix
// select (8 bits per pass, per-wave LDS histograms) finds the key tau of the
// n-th smallest and how many tau-valued elements to take; a block-wide scan of
// per-thread counts over contiguous chunks then writes the selected indices in
// ascending order (equal keys: lowest index first).
namespace {
__device__ __forceinline__ uint32_t order_key(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0xFFFFFFFFu;  // NaN sorts after +inf
    if (u == 0x80000000u) u = 0u;                             // -0 == +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
constexpr uint32_t kKeyInf = 0xFF800000u;  // order_key(+inf)
}  // namespace

__global__ __launch_bounds__(1024) void select_kernel(const float *scores, int64_t len, int64_t n, int64_t pf,
                                                      int64_t pl, int64_t *out) {
    __shared__ uint32_t hist[16][256];
    __shared__ uint32_t tot[256];
    __shared__ uint32_t cnt_lt[1024], cnt_eq[1024];
    __shared__ uint32_t s_prefix, s_k;
    const int tid = threadIdx.x, wave = tid >> 6;
    const float *srow = scores + (int64_t)blockIdx.x * len;
    int64_t *orow = out + (int64_t)blockIdx.x * n;
    const int64_t rec = len - pl > 0 ? len - pl : 0;
    auto key = [&](int64_t i) -> uint32_t { return (i < pf || i >= rec) ? kKeyInf : order_key(srow[i]); };
    if (tid == 0) {
        s_prefix = 0u;
        s_k = (uint32_t)n;  // rank (1-based) of the key to find among the remaining candidates
    }
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int i = tid; i < 16 * 256; i += 1024) (&hist[0][0])[i] = 0u;
        __syncthreads();
        const uint32_t prefix = s_prefix;
        const uint32_t hmask = pass == 0 ? 0u : (0xFFFFFFFFu << (shift + 8));
        for (int64_t i = tid; i < len; i += 1024) {
            const uint32_t k = key(i);
            if ((k & hmask) == prefix) atomicAdd(&hist[wave][(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 256) {
            uint32_t t = 0;
#pragma unroll
            for (int w = 0; w < 16; ++w) t += hist[w][tid];
            tot[tid] = t;
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t k = s_k, cum = 0;
            int b = 0;
            for (; b < 255; ++b) {
                if (cum + tot[b] >= k) break;
                cum += tot[b];
            }
            s_k = k - cum;
            s_prefix = prefix | ((uint32_t)b << shift);
        }
        __syncthreads();
    }
    const uint32_t tau = s_prefix, take_eq = s_k;  // take the first take_eq elements equal to tau
    // per-thread contiguous chunk counts, then exclusive scans
    const int64_t chunk = (len + 1023) / 1024;
    const int64_t c0 = (int64_t)tid * chunk, c1 = c0 + chunk < len ? c0 + chunk : len;
    uint32_t lt = 0, eq = 0;
    for (int64_t i = c0; i < c1; ++i) {
        const uint32_t k = key(i);
        lt += k < tau;
        eq += k == tau;
    }
    cnt_lt[tid] = lt;
    cnt_eq[tid] = eq;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {  // inclusive scans (Hillis-Steele)
        const uint32_t a = tid >= off ? cnt_lt[tid - off] : 0u, e = tid >= off ? cnt_eq[tid - off] : 0u;
        __syncthreads();
        cnt_lt[tid] += a;
        cnt_eq[tid] += e;
        __syncthreads();
    }
    uint32_t lt_before = cnt_lt[tid] - lt, eq_before = cnt_eq[tid] - eq;
    for (int64_t i = c0; i < c1; ++i) {
        const uint32_t k = key(i);
        if (k < tau) {
            const uint32_t pos = lt_before + (eq_before < take_eq ? eq_before : take_eq);
            orow[pos] = i;
            ++lt_before;
        } else if (k == tau) {
            if (eq_before < take_eq) orow[lt_before + eq_before] = i;
            ++eq_before;
        }
    }
}

// Rows of up to 65536 scores: the same selection with the keys read once and
// kept on chip (element tid + 1024 j in slot j of thread tid): slots 0-31 in
// registers, slots 32-63 in LDS (128 KiB, one 4 KiB row per slot, so a slot's
// reads are conflict-free) -- all 64 in registers spilled 30 VGPRs to scratch at
// 1024 threads.  In the first pass (sign and exponent bits, which cluster) the two
// most common digits of a wave are added as groups (one LDS atomic each) before the
// per-lane atomics; the digit searches and the output positions use wave scans (the
// positions from per-(slot, wave) counts scanned in element order).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = (uint32_t)__shfl_up((int)x, o);
        if (lane >= o) x += y;
    }
    return x;
}
constexpr int kSelSlots = 64, kSelRegSlots = 32;
// dynamic LDS of select_reg_kernel: hist[16][256], tot[256], cnt_lt[1024], cnt_eq[1024],
// s_prefix, s_k (padded to 16 bytes), then the LDS key slots [32][1024]
constexpr int kSelLdsWords = 16 * 256 + 256 + 2 * 1024 + 4 + (kSelSlots - kSelRegSlots) * 1024;
constexpr int kSelLdsBytes = kSelLdsWords * 4;
static_assert(kSelLdsBytes <= 160 * 1024, "select keys exceed the LDS");
__global__ __launch_bounds__(1024) void select_reg_kernel(const float *scores, int64_t len, int64_t n, int64_t pf,
                                                          int64_t pl, int64_t *out) {
    extern __shared__ __align__(16) uint32_t sel_lds[];
    uint32_t(*hist)[256] = (uint32_t(*)[256])sel_lds;
    uint32_t *tot = sel_lds + 16 * 256;
    uint32_t *cnt_lt = tot + 256, *cnt_eq = cnt_lt + 1024;
    uint32_t &s_prefix = cnt_eq[1024], &s_k = cnt_eq[1025];
    uint32_t *key_lds = cnt_eq + 1024 + 4;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const float *srow = scores + (int64_t)blockIdx.x * len;
    int64_t *orow = out + (int64_t)blockIdx.x * n;
    const int64_t rec = len - pl > 0 ? len - pl : 0;
    uint32_t key_reg[kSelRegSlots];
    // buffer loads: the slot offset is a constant, so no per-slot address registers
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(srow, (uint32_t)(len * 4));
    // 32-bit position arithmetic against per-thread limits (len <= 65536), so that no
    // per-slot index stays live in a register
    const int lim = (int)len - tid, lim_pf = (int)pf - tid, lim_rec = (int)rec - tid;
    auto to_key = [&](int j, uint32_t raw) {
        const bool prot = 1024 * j < lim_pf || 1024 * j >= lim_rec;
        return 1024 * j < lim ? (prot ? kKeyInf : order_key(__builtin_bit_cast(float, raw))) : 0u;
    };
#pragma unroll
    for (int j = 0; j < kSelRegSlots; ++j)
        key_reg[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, (uint32_t)tid * 4u, 4096 * j, 0);
#pragma unroll
    for (int j0 = kSelRegSlots; j0 < kSelSlots; j0 += 8) {  // LDS slots, 8 loads in flight at a time
        uint32_t raw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) raw[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (uint32_t)tid * 4u, 4096 * (j0 + i), 0);
#pragma unroll
        for (int i = 0; i < 8; ++i) key_lds[(j0 + i - kSelRegSlots) * 1024 + tid] = to_key(j0 + i, raw[i]);
    }
#pragma unroll
    for (int j = 0; j < kSelRegSlots; ++j) key_reg[j] = to_key(j, key_reg[j]);
    // slot j of this thread (j a compile-time constant after unrolling); a thread reads
    // only its own LDS slots, so they need no barrier
    auto key = [&](int j) -> uint32_t { return j < kSelRegSlots ? key_reg[j] : key_lds[(j - kSelRegSlots) * 1024 + tid]; };
    auto valid = [&](int j) { return 1024 * j < lim; };
    if (tid == 0) {
        s_prefix = 0u;
        s_k = (uint32_t)n;
    }
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int i = tid; i < 16 * 256; i += 1024) (&hist[0][0])[i] = 0u;
        __syncthreads();
        const uint32_t prefix = s_prefix;
        const uint32_t hmask = pass == 0 ? 0u : (0xFFFFFFFFu << (shift + 8));
#pragma unroll
        for (int j = 0; j < kSelSlots; ++j) {
            const uint32_t d = (key(j) >> shift) & 255u;
            bool pend = valid(j) && (key(j) & hmask) == prefix;
            if (pass == 0) {  // the sign / exponent digit clusters: add the two most common
                              // digits of the wave as groups, the rest per lane
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const uint64_t act = __builtin_amdgcn_ballot_w64(pend);
                    if (!act) break;
                    const int first = (int)__builtin_ctzll(act);
                    const uint32_t db = (uint32_t)__builtin_amdgcn_readlane((int)d, first);
                    const uint64_t m = __builtin_amdgcn_ballot_w64(pend && d == db);
                    if (lane == first) atomicAdd(&hist[wave][db], (uint32_t)__builtin_popcountll(m));
                    pend = pend && d != db;
                }
            }
            if (pend) atomicAdd(&hist[wave][d], 1u);
            asm volatile("" ::: "memory");
        }
        __syncthreads();
        // digit of the k-th key: scan of the 256 bin totals (4 waves), then the one
        // bin with excl < k <= incl (the last bin also when the keys run out)
        const uint32_t k = s_k;
        uint32_t t = 0, incl = 0;
        if (tid < 256) {
#pragma unroll
            for (int w = 0; w < 16; ++w) t += hist[w][tid];
            incl = wave_incl_scan(t, lane);
            if (lane == 63) tot[wave] = incl;
        }
        __syncthreads();
        if (tid < 256) {
            for (int w = 0; w < wave; ++w) incl += tot[w];
            const uint32_t excl = incl - t;
            if (excl < k && (k <= incl || tid == 255)) {
                s_k = k - excl;
                s_prefix = prefix | ((uint32_t)tid << shift);
            }
        }
        __syncthreads();
    }
    const uint32_t tau = s_prefix, take_eq = s_k;  // take the first take_eq elements equal to tau
    // counts of (slot j, wave w) at entry 16 j + w: element order
#pragma unroll
    for (int j = 0; j < kSelSlots; ++j) {
        const uint64_t ml = __builtin_amdgcn_ballot_w64(valid(j) && key(j) < tau);
        const uint64_t me = __builtin_amdgcn_ballot_w64(valid(j) && key(j) == tau);
        if (lane == 0) {
            cnt_lt[16 * j + wave] = (uint32_t)__builtin_popcountll(ml);
            cnt_eq[16 * j + wave] = (uint32_t)__builtin_popcountll(me);
        }
        asm volatile("" ::: "memory");
    }
    __syncthreads();
    {  // exclusive scans of the 1024 counts: in each wave, then across the 16 waves
        const uint32_t own_lt = cnt_lt[tid], own_eq = cnt_eq[tid];
        uint32_t il = wave_incl_scan(own_lt, lane), ie = wave_incl_scan(own_eq, lane);
        if (lane == 63) {
            hist[0][wave] = il;
            hist[1][wave] = ie;
        }
        __syncthreads();
        for (int w = 0; w < wave; ++w) {
            il += hist[0][w];
            ie += hist[1][w];
        }
        cnt_lt[tid] = il - own_lt;
        cnt_eq[tid] = ie - own_eq;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kSelSlots; ++j) {
        const bool lt = valid(j) && key(j) < tau, eq = valid(j) && key(j) == tau;
        const uint64_t ml = __builtin_amdgcn_ballot_w64(lt), me = __builtin_amdgcn_ballot_w64(eq);
        const uint32_t lt_before = cnt_lt[16 * j + wave] + __builtin_amdgcn_mbcnt_hi((uint32_t)(ml >> 32),
                                       __builtin_amdgcn_mbcnt_lo((uint32_t)ml, 0u));
        const uint32_t eq_before = cnt_eq[16 * j + wave] + __builtin_amdgcn_mbcnt_hi((uint32_t)(me >> 32),
                                       __builtin_amdgcn_mbcnt_lo((uint32_t)me, 0u));
        const int64_t i = (int64_t)(tid + 1024 * j);
        if (lt) orow[lt_before + (eq_before < take_eq ? eq_before : take_eq)] = i;
        else if (eq && eq_before < take_eq) orow[lt_before + eq_before] = i;
        asm volatile("" ::: "memory");  // one slot at a time (keeps the live ranges short)
    }
}

hipError_t select_launch(const float *scores, int64_t rows, int64_t len, int64_t n, int64_t pf, int64_t pl,
                         int64_t *out, hipStream_t s) {
    if (rows <= 0 || n <= 0) return hipSuccess;
    if (len <= 1024 * kSelSlots) {
        // raise the dynamic LDS cap above 64 KiB once per device (a bit per device index;
        // host threads that race here both set it, which is harmless)
        static std::atomic<uint64_t> attr_devs{0};
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        const uint64_t bit = (dev >= 0 && dev < 64) ? 1ull << dev : 0ull;
        if (!bit || !(attr_devs.load(std::memory_order_acquire) & bit)) {
            e = hipFuncSetAttribute((const void *)select_reg_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    kSelLdsBytes);
            if (e != hipSuccess) return e;
            attr_devs.fetch_or(bit, std::memory_order_release);
        }
        hipLaunchKernelGGL(select_reg_kernel, dim3((unsigned)rows), dim3(1024), kSelLdsBytes, s, scores, len, n, pf,
                           pl, out);
    }
    else
        hipLaunchKernelGGL(select_kernel, dim3((unsigned)rows), dim3(1024), 0, s, scores, len, n, pf, pl, out);
    return hipGetLastError();
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
__global__ void zero_fill_kernel(u4 *p, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = (u4){0u, 0u, 0u, 0u};
}
hipError_t zero_fill_launch(void *p, int64_t bytes, hipStream_t s) {
    const int64_t n16 = bytes / 16;
    if (n16 <= 0) return hipSuccess;
    const int64_t blocks = (n16 + 255) / 256;
    hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, s, (u4 *)p, n16);
    return hipGetLastError();
}
// Streaming read of `bytes` (a multiple of 16) in 16-byte non-temporal loads over a
// grid-stride loop, the loads XORed into a value that is stored only if it equals a
// sentinel: the bandwidth a read-once kernel of that size reaches on this GPU.
__global__ __launch_bounds__(256) void stream_read_kernel(const u4 *__restrict__ x, int64_t n16, uint32_t *sink) {
    u4 acc = {0u, 0u, 0u, 0u};
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        acc ^= __builtin_nontemporal_load(x + i);
    const uint32_t r = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (r == 0x5A17C0DEu) sink[0] = r;
}
hipError_t stream_read_launch(const void *p, int64_t bytes, uint32_t *sink, hipStream_t s) {
    const int64_t n16 = bytes / 16;
    if (n16 <= 0) return hipSuccess;
    // 2048 workgroups of 256 threads: the fastest of 1024-8192 for 73 MB - 1 GB reads
    hipLaunchKernelGGL(stream_read_kernel, dim3(2048), dim3(256), 0, s, (const u4 *)p, n16, sink);
    return hipGetLastError();
}
hipError_t importance_launch(const ImportanceParams &p, hipStream_t s) {
    if (p.n_scores == 0) return hipSuccess;
    if (p.pool <= 1) {
        const unsigned tiles = (unsigned)((p.n_scores + kImpKeys - 1) / kImpKeys);
        const int64_t rows = p.B * p.H * (p.M - p.m0);
        if (tiles >= 512 || rows < 64) hipLaunchKernelGGL(importance_rows_kernel<4>, dim3(tiles), dim3(256), 0, s, p);
        else hipLaunchKernelGGL(importance_rows_kernel<16>, dim3(tiles), dim3(1024), 0, s, p);
    } else {
        hipLaunchKernelGGL(importance_kernel, dim3((unsigned)((p.n_scores + 255) / 256)), dim3(256), 0, s, p);
    }
    return hipGetLastError();
}

}  // namespace akv
