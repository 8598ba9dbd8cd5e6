// Split-K fused dequant-attention over a hot fp16 + warm packed KV cache.
//
// Grid: (split, kv-head, batch * row-chunk).  A workgroup (4 waves) owns one
// (batch, kv-head) and one contiguous token range of either the warm or the
// hot segment.  Its query rows are the Hq/Hkv query heads (x M query
// positions) that share the kv head -- up to 16 rows, the N dimension of the
// matrix-core tiles, so every K/V byte loaded feeds all of them.
//
// Per 16-token tile a wave does:
//   QK:  S^T[16 tok x 16 rows] = K_tile . Q^T with 16x16x32 f16 MFMA.  Lane
//        (token l%16, group l/16) dequantizes D/4 channels of its token
//        straight from the packed row into the A operand.  Codes are moved
//        into fp16 halves with byte permutes and one and-or against the
//        0x6400 exponent; a code sitting 2^o above bit 0 is multiplied by a
//        block scale pre-divided by 2^o (exact whenever that scale is
//        representable, checked per block; otherwise codes are shifted down).
//        The Q operand is permuted to the channel order the codes come out in.
//   softmax: online in the log2 domain with a lazy rescale (only when a row
//        max grows by more than 8); probabilities enter the PV product as
//        fp16 scaled by 2^7.
//   PV:  O^T[16 chunks x 16 rows] += V^T . P^T with 16x16x16 f16 MFMA.  Lane
//        (chunk l%16, tokens 4*(l/16)..+3) reads one 8-channel chunk of 4
//        tokens and forms (token, token) half pairs.
// Loads of tile i+1 (codes and scale/zero) are issued before tile i is
// computed.  Waves merge in LDS; one (m, l, acc) partial per workgroup goes to
// the workspace and decode_reduce_kernel merges the splits (log-sum-exp).
#include "akv_common.h"
#include "decode.h"

namespace akv {

constexpr float kThresh = 8.0f;    // lazy-rescale threshold (log2 units)
constexpr float kPLog2 = 7.0f;     // fp16 probabilities carry a 2^7 factor
constexpr int kNW = 4;             // waves per workgroup

__device__ __forceinline__ float wave_max16(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}
__device__ __forceinline__ float wave_sum16(float x) {
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

// (x & m) | c in one VALU op (GFX9 VOP3 takes no literals, so the compiler
// otherwise splits it into and + or).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(m), "s"(c));
    return r;
}

constexpr uint32_t kMagic = 0x64006400u;

// ---------------------------------------------------------------------------
// K side (lane = one token, LCH = D/4 channels).  Pair pi of the lane's codes
// lives in a window dword at bit offset koff (both halves); its channels are
// kpair_chan<KB>(pi, 0/1).
// ---------------------------------------------------------------------------
template <int KB>
__host__ __device__ constexpr int koff(int pi) {
    if (KB == 3) {
        return (pi % 8) == 0 ? 0 : (pi % 8) == 1 ? 3 : (pi % 8) == 2 ? 6 : (pi % 8) == 3 ? 1
             : (pi % 8) == 4 ? 4 : (pi % 8) == 5 ? 7 : (pi % 8) == 6 ? 2 : 5;
    } else if (KB == 4) {
        return (pi % 2) * 4;
    } else if (KB == 2) {
        return 2 * (pi % 4);
    }
    return 0;
}

// windows: 3-bit -> 3 per word pair, 4-bit / 2-bit -> 2 per dword
template <int KB>
struct KWin {
    uint32_t w[(KB == 3) ? 6 : (KB == 4 ? 8 : 4)];
};

template <int KB, int NP>
__device__ __forceinline__ void k_windows(const uint32_t *r, KWin<KB> &W) {
    if (KB == 3) {
        // word pair 0: bytes b0..b5 (r0 = b0..b3, r1 = b4..b7); pair 1: b6..b11
        W.w[0] = perm(r[1], r[0], 0x04050102u);  // [b2 b1 | b5 b4]  W[15:0]
        W.w[1] = perm(r[1], r[0], 0x03040001u);  // [b1 b0 | b4 b3]  W[23:8]
        W.w[2] = perm(r[1], r[0], 0x0C030C00u);  // [b0 0  | b3 0 ]  W[23:16]
        if (NP > 8) {
            W.w[3] = perm(r[2], r[1], 0x06070304u);
            W.w[4] = perm(r[2], r[1], 0x05060203u);
            W.w[5] = perm(r[2], r[1], 0x0C050C02u);
        }
    } else if (KB == 4) {
#pragma unroll
        for (int d = 0; d < NP / 4; ++d) {
            W.w[2 * d] = r[d];                               // bytes 0 | 2
            W.w[2 * d + 1] = perm(0u, r[d], 0x0C030C01u);   // bytes 1 | 3
        }
    } else if (KB == 2) {
#pragma unroll
        for (int d = 0; d < NP / 8; ++d) {
            W.w[2 * d] = r[d];
            W.w[2 * d + 1] = perm(0u, r[d], 0x0C030C01u);
        }
    }
}

template <int KB>
__device__ __forceinline__ uint32_t k_window_of(const KWin<KB> &W, int pi) {
    if (KB == 3) {
        const int k = pi % 8, base = 3 * (pi / 8);
        return W.w[base + (k < 3 ? 0 : (k < 6 ? 1 : 2))];
    } else if (KB == 4) {
        return W.w[2 * (pi / 4) + ((pi % 4) >= 2 ? 1 : 0)];
    } else {
        return W.w[2 * (pi / 8) + ((pi % 8) >= 4 ? 1 : 0)];
    }
}

template <int KB>
__host__ __device__ constexpr uint32_t kmask(int pi) {
    return (((KB == 3) ? 7u : (KB == 4 ? 15u : 3u)) << koff<KB>(pi)) * 0x00010001u;
}

// ---------------------------------------------------------------------------
struct WaveState {
    float m2;      // running max of this lane's row (log2 domain: q.k * sm_scale * log2 e)
    float l;       // partial sum of 2^7 * exp2(s - m2) over this lane's tokens
    f4 acc[8];     // O^T: acc[j][i] = chunk (4*grp+i), channel slot j, row col (x 2^7)
};

// online softmax over one tile.  s: raw q.k for tokens 4*grp+i of row col.
// Returns the fp16 P^T operand (x 2^7); rescales the running state when needed.
__device__ __forceinline__ h4 softmax_tile(WaveState &st, f4 s, float sl2) {
    float t = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    t = wave_max16(t);
    const float tm2 = t * sl2;
    if (__builtin_amdgcn_ballot_w64(tm2 > st.m2 + kThresh)) {  // wave-uniform, rare after warm-up
        const float mn = fmaxf(st.m2, tm2);
        const float alpha = __builtin_amdgcn_exp2f(st.m2 - mn);
        st.l *= alpha;
#pragma unroll
        for (int j = 0; j < 8; ++j) st.acc[j] *= alpha;
        st.m2 = mn;
    }
    const float bias = kPLog2 - st.m2;
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], sl2, bias));
    st.l += (p[0] + p[1]) + (p[2] + p[3]);
    return (h4){(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
}

// The stash holds the raw logits q.k; its readers take them to the log2 domain with
// the softmax's own fma, 2^(x sl2 - M) (one rounding).
__device__ __forceinline__ void store_stash(const DecodeParams &p, int64_t rowbase, int row_valid, int64_t nlog0,
                                            f4 s, int nvalid) {
    if (!p.stash || !row_valid) return;
    float *dst = p.stash + rowbase + nlog0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (i < nvalid) dst[i] = s[i];
}

// raw loads of one warm tile
template <int D, int KB, int VB, int WK>
struct WarmRaw {
    static constexpr int KBYTES = (D / 4) * KB / 8;
    static constexpr int KDW = (KBYTES + 3) / 4;
    uint32_t k[KDW];
    uint32_t v[4][VB == 8 ? 2 : 1];
    uint32_t ms[4], mz[4];  // V meta staging values (fp16 bits or fp32 bits)
    float lks[4], lkz[4];   // legacy K meta of this lane's token
};

template <int D, int KB, int VB, int WK>
__device__ __forceinline__ void load_warm_tile(WarmRaw<D, KB, VB, WK> &R, const DecodeParams &p, int t0, int lane,
                                               int col, int grp, __amdgpu_buffer_rsrc_t rkc,
                                               __amdgpu_buffer_rsrc_t rvc, __amdgpu_buffer_rsrc_t rvs,
                                               __amdgpu_buffer_rsrc_t rvz, int ngr, int nwarm, int64_t hw) {
    constexpr int LCH = D / 4;
    constexpr int KBYTES = WarmRaw<D, KB, VB, WK>::KBYTES;
    constexpr int VCH = D / 8;
    // K codes: lane's token t0+col, channels LCH*grp .. +LCH
    {
        const uint32_t off = (uint32_t)(t0 + col) * (uint32_t)p.kc_row + KBYTES * grp;
        if (KBYTES == 12) { u3 x = bld96(rkc, off); R.k[0] = x[0]; R.k[1] = x[1]; R.k[2] = x[2]; }
        else if (KBYTES == 16) { u4 x = bld128(rkc, off); R.k[0] = x[0]; R.k[1] = x[1]; R.k[2] = x[2]; R.k[3] = x[3]; }
        else if (KBYTES == 8) { u2 x = bld64(rkc, off); R.k[0] = x[0]; R.k[1] = x[1]; }
        else if (KBYTES == 6) {  // 3-bit, D=64: 6 bytes at a 2-byte-aligned offset
            const uint32_t base = off & ~3u;
            const int sh = (int)(off - base);
            u3 x = bld96(rkc, base);
            R.k[0] = __builtin_amdgcn_alignbyte(x[1], x[0], sh);
            R.k[1] = __builtin_amdgcn_alignbyte(x[2], x[1], sh) & 0xFFFFu;
        } else if (KBYTES == 4) { R.k[0] = bld32(rkc, off); }
        else if (KBYTES == 32) {
            u4 x = bld128(rkc, off), y = bld128(rkc, off + 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) { R.k[q] = x[q]; R.k[(4 + q) % WarmRaw<D, KB, VB, WK>::KDW] = y[q]; }
        }
    }
    // V codes: chunk col of tokens t0+4*grp .. +3
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
        const uint32_t rowoff = (uint32_t)(t0 + 4 * grp + jj) * (uint32_t)p.vc_row;
        uint32_t a = 0u, bb = 0u;
        if (col < VCH) {
            if (VB == 4) a = bld32(rvc, rowoff + 4 * col);
            else if (VB == 2) a = bld16(rvc, rowoff + 2 * col);
            else if (VB == 8) { u2 x = bld64(rvc, rowoff + 8 * col); a = x[0]; bb = x[1]; }
            else {  // 3 bytes at 3*col: read the aligned 8 bytes around them
                const int off = (3 * col) & ~3;
                u2 x = bld64(rvc, rowoff + off);
                a = __builtin_amdgcn_alignbyte(x[1], x[0], 3 * col - off);
            }
        }
        R.v[jj][0] = a;
        if (VB == 8) R.v[jj][VB == 8 ? 1 : 0] = bb;
    }
    // V scale/zero of the tile's 16 tokens x ngr groups (staged through LDS at compute time)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int e = lane + 64 * i;
        R.ms[i] = 0u;
        R.mz[i] = 0u;
        if (e < 16 * ngr) {
            const int tt = e / ngr, gg = e - tt * ngr;
            const uint32_t mi = (uint32_t)(t0 + tt) * (uint32_t)ngr + gg;
            if (WK == AKV_WARM_AFFINE) {
                R.ms[i] = bld16(rvs, 2 * mi);
                R.mz[i] = bld16(rvz, 2 * mi);
            } else {
                const int tv = min(t0 + tt, nwarm - 1);
                const int64_t gi = (hw * p.w_stride + tv) * ngr + gg;
                R.ms[i] = __builtin_bit_cast(uint32_t, load_as_f32(p.vs, gi, p.meta_dt));
                R.mz[i] = __builtin_bit_cast(uint32_t, load_as_f32(p.vz, gi, p.meta_dt));
            }
        }
    }
    if (WK == AKV_WARM_LEGACY) {  // K meta of this lane's token (groups covering its channels)
        const int ng = LCH / p.gs > 0 ? LCH / p.gs : 1;
        const int64_t mrow = hw * p.w_stride + min(t0 + col, nwarm - 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            R.lks[q] = 0.f;
            R.lkz[q] = 0.f;
            if (q < ng) {
                const int gi = (LCH * grp) / p.gs + q;
                R.lks[q] = load_as_f32(p.ks, mrow * p.lg + gi, p.meta_dt);
                R.lkz[q] = load_as_f32(p.kz, mrow * p.lg + gi, p.meta_dt);
            }
        }
    }
}

// Occupancy target of the split kernel (waves per SIMD) handed to the register
// allocator; 0 leaves the choice to the compiler.
#ifndef AKV_SPLIT_WAVES_PER_EU
#define AKV_SPLIT_WAVES_PER_EU 0
#endif
#if AKV_SPLIT_WAVES_PER_EU > 0
#define AKV_SPLIT_ATTR __attribute__((amdgpu_waves_per_eu(AKV_SPLIT_WAVES_PER_EU, AKV_SPLIT_WAVES_PER_EU)))
#else
#define AKV_SPLIT_ATTR
#endif

template <int D, int KB, int VB, int WK, bool OUTL>
__global__ __launch_bounds__(256) AKV_SPLIT_ATTR void decode_split_kernel(const DecodeParams p) {
    constexpr int KSTEPS = D / 32, LCH = D / 4, NPAIRS = LCH / 2, VCH = D / 8;
    using Raw = WarmRaw<D, KB, VB, WK>;

    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int split = blockIdx.x, kvh = blockIdx.y;
    const int b = blockIdx.z / p.nchunk, chunk = blockIdx.z % p.nchunk;
    const int row0 = chunk * 16;
    const int nrows = min(16, p.R - row0);
    const bool is_warm = split < p.n_wsplit;

    const int r = row0 + col;
    const int row_valid = col < nrows;
    const int rc = row_valid ? r : row0;  // invalid rows reuse a valid query (results discarded)
    const int hq = kvh * p.g + rc / p.M, mq = rc % p.M;
    const int64_t strow = ((int64_t)(b * p.Hq + hq) * p.M + mq) * p.N;  // stash row base

    int t_begin, t_end;
    if (is_warm) {
        t_begin = split * (int)p.wsplit_len;
        t_end = min(t_begin + (int)p.wsplit_len, (int)p.n_warm);
    } else {
        t_begin = (split - p.n_wsplit) * (int)p.hsplit_len;
        t_end = min(t_begin + (int)p.hsplit_len, (int)p.n_hot);
    }
    const int64_t seg_base = is_warm ? (p.hot_first ? p.n_hot : 0) : (p.hot_first ? 0 : p.n_warm);

    // ---- Q operand (B of the QK MFMA): lane = (row col, channel group grp)
    h8 qop[KSTEPS];
    {
        const _Float16 *qrow = p.q + ((int64_t)(b * p.Hq + hq) * p.M + mq) * D + LCH * grp;
#pragma unroll
        for (int st = 0; st < KSTEPS; ++st)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int pi = 4 * st + j / 2, hf = j % 2;
                const int ch = is_warm ? kpair_chan<KB>(pi, hf) : kpair_chan<16>(pi, hf);
                qop[st][j] = qrow[ch];
            }
    }

    WaveState stt;
    stt.m2 = -INFINITY;
    stt.l = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) stt.acc[j] = (f4){0.f, 0.f, 0.f, 0.f};

    // per-wave LDS staging: K meta [s'|s|z][4 grp][16 pairs] u32 (768 B),
    // V meta [s|z][16 groups][16 tokens] of <= 4 B (2 KiB)
    uint32_t *kmeta_lds = (uint32_t *)(smem + wave * 2816);
    unsigned char *vmeta_lds = smem + wave * 2816 + 768;

    const int64_t bh = (int64_t)b * p.Hkv + kvh;
    const float sl2 = p.scale_log2;

    if (!is_warm) {
        // ------------------------------------------------------------ hot tiles
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.khot + bh * p.h_stride * D, (uint32_t)(p.n_hot * D * 2));
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.vhot + bh * p.h_stride * D, (uint32_t)(p.n_hot * D * 2));
        for (int t0 = t_begin + 16 * wave; t0 < t_end; t0 += 16 * kNW) {
            h8 kop[KSTEPS];
#pragma unroll
            for (int st = 0; st < KSTEPS; ++st) {
                u4 raw = bld128(rk, (uint32_t)(((t0 + col) * D + LCH * grp + 8 * st) * 2));
                kop[st] = __builtin_bit_cast(h8, raw);
            }
            u4 w[4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                w[jj] = (col < VCH) ? bld128(rv, (uint32_t)(((t0 + 4 * grp + jj) * D + 8 * col) * 2))
                                    : (u4){0u, 0u, 0u, 0u};
            f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < KSTEPS; ++st) s = mfma_k32(kop[st], qop[st], s);
            const int nvalid = min(4, t_end - (t0 + 4 * grp));
            if (t0 + 16 > t_end) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (i >= nvalid) s[i] = -INFINITY;
            }
            store_stash(p, strow, row_valid, seg_base + t0 + 4 * grp, s, nvalid);
            const h4 pop = softmax_tile(stt, s, sl2);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                const uint32_t lo = perm(w[1][j / 2], w[0][j / 2], sel);
                const uint32_t hi = perm(w[3][j / 2], w[2][j / 2], sel);
                stt.acc[j] = mfma_k16(__builtin_bit_cast(h4, (u2){lo, hi}), pop, stt.acc[j]);
            }
        }
    } else {
        // ----------------------------------------------------------- warm tiles
        const int unit = (WK == AKV_WARM_AFFINE) ? p.T : 16;  // tokens sharing K meta
        // legacy: one tier shared by all, one per kv head, or one per (batch, kv head)
        const int64_t hw = (WK == AKV_WARM_AFFINE) ? bh : (p.warm_heads == 1 ? 0 : p.warm_heads == p.Hkv ? kvh : bh);
        const int nwarm = (int)p.n_warm;
        const __amdgpu_buffer_rsrc_t rkc =
            make_rsrc((const unsigned char *)p.kc + hw * p.w_stride * p.kc_row, (uint32_t)(p.n_warm * p.kc_row));
        const __amdgpu_buffer_rsrc_t rvc =
            make_rsrc((const unsigned char *)p.vc + hw * p.w_stride * p.vc_row, (uint32_t)(p.n_warm * p.vc_row));
        const int ngr = (WK == AKV_WARM_AFFINE) ? D / p.Gv : p.lg;
        const __amdgpu_buffer_rsrc_t rvs =
            make_rsrc((const _Float16 *)p.vs + hw * p.w_stride * ngr, (uint32_t)(p.n_warm * ngr * 2));
        const __amdgpu_buffer_rsrc_t rvz =
            make_rsrc((const _Float16 *)p.vz + hw * p.w_stride * ngr, (uint32_t)(p.n_warm * ngr * 2));
        const __amdgpu_buffer_rsrc_t rks =
            make_rsrc((const _Float16 *)p.ks + bh * p.nblk * D, (uint32_t)(p.nblk * D * 2));
        const __amdgpu_buffer_rsrc_t rkz =
            make_rsrc((const _Float16 *)p.kz + bh * p.nblk * D, (uint32_t)(p.nblk * D * 2));
        int ksym = 0, vsym = 0;
        if (WK == AKV_WARM_LEGACY) {
            ksym = p.sym_flags ? p.sym_flags[0] : p.legacy_sym;
            vsym = p.sym_flags ? p.sym_flags[1] : p.legacy_sym;
        }
        const int gsz = (WK == AKV_WARM_AFFINE) ? p.Gv : p.gs;
        const int gme = min((8 * col) / gsz, 15);  // V group of this lane's chunk
        // K meta staging role of this lane: (group g2, pair pi2)
        const int g2 = lane >> 4, pi2 = lane & 15;
        int clo = 0, chi = 0, ko2 = 0;
#pragma unroll
        for (int q = 0; q < NPAIRS; ++q)
            if (q == pi2) { clo = kpair_chan<KB>(q, 0); chi = kpair_chan<KB>(q, 1); ko2 = koff<KB>(q); }
        const uint32_t kmo_lo = (uint32_t)(LCH * g2 + clo) * 2, kmo_hi = (uint32_t)(LCH * g2 + chi) * 2;

        Raw cur, nxt;
        uint32_t km_s = 0u, km_z = 0u;  // prefetched K meta pair (s, z) of the next unit (affine)
        int u0 = t_begin + unit * wave;
        if (u0 < t_end) {
            load_warm_tile<D, KB, VB, WK>(nxt, p, u0, lane, col, grp, rkc, rvc, rvs, rvz, ngr, nwarm, hw);
            if (WK == AKV_WARM_AFFINE && pi2 < NPAIRS) {
                const uint32_t mo = (uint32_t)(u0 / p.T) * D * 2;
                km_s = (uint32_t)bld16(rks, mo + kmo_lo) | ((uint32_t)bld16(rks, mo + kmo_hi) << 16);
                km_z = (uint32_t)bld16(rkz, mo + kmo_lo) | ((uint32_t)bld16(rkz, mo + kmo_hi) << 16);
            }
        }
        for (; u0 < t_end; u0 += unit * kNW) {
            // ---- K meta of this unit -> LDS (affine: per channel of the block, pair order)
            bool fast = true;
            if (WK == AKV_WARM_AFFINE) {
                if (pi2 < NPAIRS) {
                    const h2 sv = as_h2(km_s);
                    const _Float16 f = (_Float16)(1.0f / (float)(1 << ko2));
                    const h2 sp = sv * (h2){f, f};
                    const _Float16 gm = (_Float16)(float)(1 << ko2);
                    const h2 back = sp * (h2){gm, gm};
                    fast = (back[0] == sv[0]) && (back[1] == sv[1]);
                    kmeta_lds[(0 * 4 + g2) * 16 + pi2] = as_u32(sp);
                    kmeta_lds[(1 * 4 + g2) * 16 + pi2] = km_s;
                    kmeta_lds[(2 * 4 + g2) * 16 + pi2] = km_z;
                }
                fast = !__builtin_amdgcn_ballot_w64(!fast);
                const int nu = u0 + unit * kNW;
                if (nu < t_end && pi2 < NPAIRS) {  // prefetch the next unit's K meta
                    const uint32_t mo = (uint32_t)(nu / p.T) * D * 2;
                    km_s = (uint32_t)bld16(rks, mo + kmo_lo) | ((uint32_t)bld16(rks, mo + kmo_hi) << 16);
                    km_z = (uint32_t)bld16(rkz, mo + kmo_lo) | ((uint32_t)bld16(rkz, mo + kmo_hi) << 16);
                }
                __builtin_amdgcn_wave_barrier();
            }
            h2 ksc[NPAIRS], kze[NPAIRS];
            if (WK == AKV_WARM_AFFINE) {
                const uint32_t *src_s = kmeta_lds + ((fast ? 0 : 1) * 4 + grp) * 16;
#pragma unroll
                for (int q = 0; q < NPAIRS; ++q) {
                    ksc[q] = as_h2(src_s[q]);
                    kze[q] = as_h2(kmeta_lds[(2 * 4 + grp) * 16 + q]);
                }
            }
            const int u1 = min(u0 + unit, t_end);
            for (int t0 = u0; t0 < u1; t0 += 16) {
                cur = nxt;
                {  // prefetch the next tile of this wave
                    int tn = t0 + 16;
                    if (tn >= u1) tn = u0 + unit * kNW;
                    if (tn < t_end)
                        load_warm_tile<D, KB, VB, WK>(nxt, p, tn, lane, col, grp, rkc, rvc, rvs, rvz, ngr, nwarm, hw);
                }
                // ---- V meta of the tile -> LDS [s|z][group][token]
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int e = lane + 64 * i;
                    if (e < 16 * ngr) {
                        const int tt = e / ngr, gg = e - tt * ngr;
                        if (WK == AKV_WARM_AFFINE) {
                            ((uint16_t *)vmeta_lds)[(0 * 16 + gg) * 16 + tt] = (uint16_t)cur.ms[i];
                            ((uint16_t *)vmeta_lds)[(1 * 16 + gg) * 16 + tt] = (uint16_t)cur.mz[i];
                        } else {
                            ((uint32_t *)vmeta_lds)[(0 * 16 + gg) * 16 + tt] = cur.ms[i];
                            ((uint32_t *)vmeta_lds)[(1 * 16 + gg) * 16 + tt] = cur.mz[i];
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();
                h2 vs01, vs23, vz01, vz23;
                float fvs[4], fvz[4];
                if (WK == AKV_WARM_AFFINE) {
                    const u2 sp = *(const u2 *)((const uint16_t *)vmeta_lds + (0 * 16 + gme) * 16 + 4 * grp);
                    const u2 zp = *(const u2 *)((const uint16_t *)vmeta_lds + (1 * 16 + gme) * 16 + 4 * grp);
                    vs01 = as_h2(sp[0]); vs23 = as_h2(sp[1]);
                    vz01 = as_h2(zp[0]); vz23 = as_h2(zp[1]);
                } else {
                    const u4 sp = *(const u4 *)((const uint32_t *)vmeta_lds + (0 * 16 + gme) * 16 + 4 * grp);
                    const u4 zp = *(const u4 *)((const uint32_t *)vmeta_lds + (1 * 16 + gme) * 16 + 4 * grp);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        // copy the element out first: bit-casting a subscripted
                        // ext-vector lvalue reads element 0 whatever the index
                        const uint32_t ws = sp[i], wz = zp[i];
                        fvs[i] = __builtin_bit_cast(float, ws);
                        fvz[i] = __builtin_bit_cast(float, wz);
                    }
                }
                __builtin_amdgcn_wave_barrier();

                // ---- K dequant + QK
                f4 s = {0.f, 0.f, 0.f, 0.f};
                if (WK == AKV_WARM_AFFINE && KB != 8) {
                    KWin<KB> W;
                    k_windows<KB, NPAIRS>(cur.k, W);
                    const h2 magic = {(_Float16)1024.0f, (_Float16)1024.0f};
                    if (fast) {
                        // the code stays 2^o above bit 0; the scale was divided by 2^o
#pragma unroll
                        for (int st = 0; st < KSTEPS; ++st) {
                            h8 a;
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                const int pi = 4 * st + k;
                                const h2 c = as_h2(and_or(k_window_of<KB>(W, pi), kmask<KB>(pi), kMagic)) - magic;
                                h2 v = c * ksc[pi];
                                v = v + kze[pi];
                                a[2 * k] = v[0];
                                a[2 * k + 1] = v[1];
                            }
                            s = mfma_k32(a, qop[st], s);
                        }
                    } else {
#pragma unroll
                        for (int st = 0; st < KSTEPS; ++st) {
                            h8 a;
#pragma unroll
                            for (int k = 0; k < 4; ++k) {
                                const int pi = 4 * st + k;
                                const uint32_t z = k_window_of<KB>(W, pi) >> koff<KB>(pi);
                                const h2 c = as_h2(and_or(z, kmask<KB>(0), kMagic)) - magic;
                                h2 v = c * ksc[pi];
                                v = v + kze[pi];
                                a[2 * k] = v[0];
                                a[2 * k + 1] = v[1];
                            }
                            s = mfma_k32(a, qop[st], s);
                        }
                    }
                } else {
#pragma unroll
                    for (int st = 0; st < KSTEPS; ++st) {
                        h8 a;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const int pi = 4 * st + k;
                            const uint32_t cp = kpair_extract<KB>(cur.k, pi);
                            const int c0 = kpair_chan<KB>(pi, 0), c1 = kpair_chan<KB>(pi, 1);
                            const int q0 = (LCH / p.gs > 0) ? c0 / p.gs : 0;
                            const int q1 = (LCH / p.gs > 0) ? c1 / p.gs : 0;
                            const float s0 = q0 == 0 ? cur.lks[0] : q0 == 1 ? cur.lks[1] : q0 == 2 ? cur.lks[2] : cur.lks[3];
                            const float s1 = q1 == 0 ? cur.lks[0] : q1 == 1 ? cur.lks[1] : q1 == 2 ? cur.lks[2] : cur.lks[3];
                            const float z0 = q0 == 0 ? cur.lkz[0] : q0 == 1 ? cur.lkz[1] : q0 == 2 ? cur.lkz[2] : cur.lkz[3];
                            const float z1 = q1 == 0 ? cur.lkz[0] : q1 == 1 ? cur.lkz[1] : q1 == 2 ? cur.lkz[2] : cur.lkz[3];
                            const float u0f = (float)(cp & 0xFFFFu), u1f = (float)(cp >> 16);
                            float d0, d1;
                            if (ksym) { d0 = (u0f - p.half_max_k) * s0; d1 = (u1f - p.half_max_k) * s1; }
                            else { d0 = u0f * s0; d0 = d0 + z0; d1 = u1f * s1; d1 = d1 + z1; }
                            a[2 * k] = (_Float16)d0;
                            a[2 * k + 1] = (_Float16)d1;
                        }
                        s = mfma_k32(a, qop[st], s);
                    }
                }
                const int nvalid = min(4, t_end - (t0 + 4 * grp));
                if (t0 + 16 > t_end) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (i >= nvalid) s[i] = -INFINITY;
                }
                // ---- K outlier channels (affine): the stored fp16 value replaces the
                // dequantized one -> add q[d_j] * (o - kdeq) to the raw dot product
                if (OUTL) {
                    const int64_t blk = t0 / p.T;
#pragma unroll 1
                    for (int j = 0; j < p.n_out; ++j) {
                        const int dj = min(max((int)p.k_oidx[((int64_t)b * p.nblk + blk) * p.n_out + j], 0), D - 1);
                        const float qd = (float)p.q[((int64_t)(b * p.Hq + hq) * p.M + mq) * D + dj];
                        const _Float16 ksj = ((const _Float16 *)p.ks)[(bh * p.nblk + blk) * D + dj];
                        const _Float16 kzj = ((const _Float16 *)p.kz)[(bh * p.nblk + blk) * D + dj];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            if (i >= nvalid) continue;
                            const int64_t t = t0 + 4 * grp + i;
                            const unsigned char *row = (const unsigned char *)p.kc + (hw * p.n_warm + t) * p.kc_row;
                            const uint32_t code = extract_code(row, dj, KB);
                            const _Float16 kd = (_Float16)((_Float16)((_Float16)code * ksj) + kzj);
                            const _Float16 od = ((const _Float16 *)p.k_odata)[(bh * p.n_warm + t) * p.n_out + j];
                            s[i] += qd * ((float)od - (float)kd);
                        }
                    }
                }
                store_stash(p, strow, row_valid, seg_base + t0 + 4 * grp, s, nvalid);

                const h4 pop = softmax_tile(stt, s, sl2);
                // ---- V dequant (4 tokens x 8 channels of chunk col) + PV per channel slot
                int vo_dj[2] = {-1, -1};  // outlier channels of this block in this lane's chunk (first two)
                if (OUTL) {
                    const int64_t blk = t0 / p.T;
                    int cnt = 0;
#pragma unroll 1
                    for (int j = 0; j < p.n_out && cnt < 2; ++j) {
                        const int dj = min(max((int)p.v_oidx[((int64_t)b * p.nblk + blk) * p.n_out + j], 0), D - 1);
                        if (dj / 8 == col) vo_dj[cnt++] = j;
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    uint32_t c01, c23;
                    if (VB == 3) {
                        const uint32_t sel = j < 5 ? 0x05060102u : 0x04050001u;
                        const int sh = j < 5 ? 3 * j : 7 + 3 * (j - 5);
                        c01 = perm(cur.v[1][0], cur.v[0][0], sel) >> sh;
                        c23 = perm(cur.v[3][0], cur.v[2][0], sel) >> sh;
                    } else if (VB == 4) {
                        const uint32_t sel = j < 4 ? 0x05040100u : 0x07060302u;
                        c01 = perm(cur.v[1][0], cur.v[0][0], sel) >> (4 * (j & 3));
                        c23 = perm(cur.v[3][0], cur.v[2][0], sel) >> (4 * (j & 3));
                    } else if (VB == 2) {
                        c01 = ((cur.v[0][0] & 0xFFFFu) | (cur.v[1][0] << 16)) >> (2 * j);
                        c23 = ((cur.v[2][0] & 0xFFFFu) | (cur.v[3][0] << 16)) >> (2 * j);
                    } else {  // 8-bit: byte j%4 of dword j/4
                        constexpr int VW = (VB == 8) ? 2 : 1;
                        const int dw = (j / 4) % VW;
                        const uint32_t sel = (uint32_t)((j & 3) | (0x0C << 8) | ((4 + (j & 3)) << 16) | (0x0C << 24));
                        c01 = perm(cur.v[1][dw], cur.v[0][dw], sel);
                        c23 = perm(cur.v[3][dw], cur.v[2][dw], sel);
                    }
                    const uint32_t vm =
                        (VB == 3) ? 0x00070007u : (VB == 4 ? 0x000F000Fu : (VB == 2 ? 0x00030003u : 0x00FF00FFu));
                    c01 = and_or(c01, vm, kMagic);
                    c23 = and_or(c23, vm, kMagic);
                    const h2 magic = {(_Float16)1024.0f, (_Float16)1024.0f};
                    h2 a01, a23;
                    if (WK == AKV_WARM_AFFINE) {
                        a01 = (as_h2(c01) - magic) * vs01;
                        a01 = a01 + vz01;
                        a23 = (as_h2(c23) - magic) * vs23;
                        a23 = a23 + vz23;
                    } else {
                        const h2 x01 = as_h2(c01) - magic, x23 = as_h2(c23) - magic;
                        const float u[4] = {(float)x01[0], (float)x01[1], (float)x23[0], (float)x23[1]};
                        float d[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            if (vsym) d[i] = (u[i] - p.half_max_v) * fvs[i];
                            else { d[i] = u[i] * fvs[i]; d[i] = d[i] + fvz[i]; }
                        }
                        a01 = (h2){(_Float16)d[0], (_Float16)d[1]};
                        a23 = (h2){(_Float16)d[2], (_Float16)d[3]};
                    }
                    h4 vop = {a01[0], a01[1], a23[0], a23[1]};
                    if (OUTL && vo_dj[0] >= 0) {  // rare: outlier channels replace values
#pragma unroll
                        for (int q = 0; q < 2; ++q) {
                            const int jo = vo_dj[q];
                            if (jo < 0) continue;
                            const int dj = (int)p.v_oidx[((int64_t)b * p.nblk + t0 / p.T) * p.n_out + jo];
                            if (vpair_chan<VB>(j) != dj % 8) continue;
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const int64_t tv = min(t0 + 4 * grp + i, nwarm - 1);
                                vop[i] = ((const _Float16 *)p.v_odata)[(bh * p.n_warm + tv) * p.n_out + jo];
                            }
                        }
                    }
                    stt.acc[j] = mfma_k16(vop, pop, stt.acc[j]);
                }
            }
        }
    }

    // ---- merge the waves of this workgroup, write the split partial
    stt.l = wave_sum16(stt.l);
    __syncthreads();
    float *mlds = (float *)smem;                   // [NW][16] max
    float *llds = mlds + kNW * 16;                 // [NW][16] sum
    float *alds = llds + kNW * 16;                 // [NW][16][D] acc
    if (grp == 0) {
        mlds[wave * 16 + col] = stt.m2;
        llds[wave * 16 + col] = stt.l;
    }
    const int vperm_hot = !is_warm;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int chunkrow = 4 * grp + i;
            if (chunkrow < VCH) {
                const int ch = 8 * chunkrow + (vperm_hot ? j : vpair_chan<VB>(j));
                alds[(wave * 16 + col) * D + ch] = stt.acc[j][i];
            }
        }
    __syncthreads();
    float *part = p.part + ((bh * p.nchunk + chunk) * p.nsplit + split) * (int64_t)(p.prows * (D + 4));
    for (int e = threadIdx.x; e < nrows * D; e += 256) {
        const int rr = e / D, ch = e % D;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kNW; ++w) mx = fmaxf(mx, mlds[w * 16 + rr]);
        float a = 0.f, l = 0.f;
#pragma unroll
        for (int w = 0; w < kNW; ++w) {
            const float mw = mlds[w * 16 + rr];
            const float f = (mw == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mw - mx);
            a += f * alds[(w * 16 + rr) * D + ch];
            l += f * llds[w * 16 + rr];
        }
        part[rr * (D + 4) + 4 + ch] = a;
        if (ch == 0) {
            part[rr * (D + 4) + 0] = mx;
            part[rr * (D + 4) + 1] = l;
        }
    }
}

// Merge the split partials of one query row: out = sum_s f_s acc_s / sum_s f_s l_s,
// f_s = exp2(m_s - M).  One workgroup of 256 threads per (batch, kv-head, chunk,
// row): thread = (channel quad q, split lane sl); each thread keeps its splits'
// float4 loads in flight, the split lanes are summed through LDS.
// Merge the split partials (m, l, acc) of one query row: row rr of 16-row
// chunk bhc % nchunk of (batch, kv-head) bhc / nchunk, into the output (and
// the row statistics when p.rowstats).  Thread (split lane sl, channel quad
// q) walks splits sl, sl + SL, ... in batches of KB whose loads are all in
// flight together, merging them online (log-sum-exp); the SL lanes then merge
// through LDS.  At <= SL*KB splits the whole merge costs one round trip to
// memory.  256 threads.
template <int D>
__device__ __forceinline__ void merge_split_row(const DecodeParams &p, int bhc, int rr, float *sm, float *sls,
                                                f4 (*accl)[D / 4]) {
    constexpr int NQ = D / 4, SL = 256 / NQ, PS = D + 4, KB = 4;
    const int chunk = bhc % p.nchunk;
    const int64_t bh = bhc / p.nchunk;
    const int b = (int)(bh / p.Hkv), kvh = (int)(bh % p.Hkv);
    const int row0 = chunk * 16, nrows = min(16, p.R - row0);
    if (rr >= nrows) return;
    const int ns = p.nsplit;
    const int64_t pstride = (int64_t)p.prows * PS;
    const float *part = p.part + (bh * p.nchunk + chunk) * (int64_t)ns * pstride + rr * PS;
    const int tid = threadIdx.x, q = tid % NQ, sl = tid / NQ;
    float mx = -INFINITY, l = 0.f;
    f4 a = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = sl; s0 < ns; s0 += KB * SL) {
        float ms[KB], ls[KB];
        f4 xs[KB];
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            const int s = s0 + k * SL;
            if (s < ns) {
                ms[k] = part[s * pstride];
                ls[k] = part[s * pstride + 1];
                xs[k] = *(const f4 *)(part + s * pstride + 4 + 4 * q);
            } else {
                ms[k] = -INFINITY;
                ls[k] = 0.f;
                xs[k] = (f4){0.f, 0.f, 0.f, 0.f};
            }
        }
        float nm = mx;
#pragma unroll
        for (int k = 0; k < KB; ++k) nm = fmaxf(nm, ms[k]);
        if (nm == -INFINITY) continue;
        const float fo = (mx == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(mx - nm);
        a *= fo;
        l *= fo;
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            const float f = (ms[k] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ms[k] - nm);
            a += f * xs[k];
            l += f * ls[k];
        }
        mx = nm;
    }
    if (q == 0) {
        sm[sl] = mx;
        sls[sl] = l;
    }
    accl[sl][q] = a;
    __syncthreads();
    if (tid < NQ) {
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < SL; ++k) M = fmaxf(M, sm[k]);
        f4 o = {0.f, 0.f, 0.f, 0.f};
        float L = 0.f;
#pragma unroll
        for (int k = 0; k < SL; ++k) {
            const float f = (sm[k] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(sm[k] - M);
            o += f * accl[k][tid];
            L += f * sls[k];
        }
        const int r = row0 + rr;
        const int h = kvh * p.g + r / p.M, m = r % p.M;
        const int64_t row = (int64_t)(b * p.Hq + h) * p.M + m;
        if (p.out_bf16) {
            const u2 ov = {(uint32_t)f32_to_bf16_rne(o[0] / L) | ((uint32_t)f32_to_bf16_rne(o[1] / L) << 16),
                           (uint32_t)f32_to_bf16_rne(o[2] / L) | ((uint32_t)f32_to_bf16_rne(o[3] / L) << 16)};
            *(u2 *)(p.out + row * D + 4 * tid) = ov;
        } else {
            const h4 ov = {(_Float16)(o[0] / L), (_Float16)(o[1] / L), (_Float16)(o[2] / L), (_Float16)(o[3] / L)};
            *(h4 *)(p.out + row * D + 4 * tid) = ov;
        }
        if (tid == 0 && p.rowstats) {
            p.rowstats[2 * row] = M;
            p.rowstats[2 * row + 1] = 1.0f / (L * (1.0f / 128.0f));  // 1 / L, the 2^7 probability scale undone
        }
    }
}

// Few splits (<= 8, chunked prefill): thread = (row of the chunk, channel quad)
// with all its split loads in flight; 256 / (D/4) rows per workgroup.
template <int D>
__global__ __launch_bounds__(256) void reduce_few_kernel(const DecodeParams p) {
    constexpr int NQ = D / 4, RPW = 256 / NQ, PS = D + 4, KS = 8;
    const int bhc = blockIdx.x;
    const int rr = blockIdx.y * RPW + threadIdx.x / NQ, q = threadIdx.x % NQ;
    const int chunk = bhc % p.nchunk;
    const int64_t bh = bhc / p.nchunk;
    const int b = (int)(bh / p.Hkv), kvh = (int)(bh % p.Hkv);
    const int row0 = chunk * 16, nrows = min(16, p.R - row0);
    if (rr >= nrows) return;
    const int ns = p.nsplit;
    const int64_t pstride = (int64_t)p.prows * PS;
    const float *part = p.part + (bh * p.nchunk + chunk) * (int64_t)ns * pstride + rr * PS;
    float ms[KS], ls[KS];
    f4 xs[KS];
#pragma unroll
    for (int k = 0; k < KS; ++k) {
        const bool in = k < ns;
        ms[k] = in ? part[k * pstride] : -INFINITY;
        ls[k] = in ? part[k * pstride + 1] : 0.f;
        xs[k] = in ? *(const f4 *)(part + k * pstride + 4 + 4 * q) : (f4){0.f, 0.f, 0.f, 0.f};
    }
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < KS; ++k) M = fmaxf(M, ms[k]);
    f4 o = {0.f, 0.f, 0.f, 0.f};
    float L = 0.f;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
        const float f = (ms[k] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ms[k] - M);
        o += f * xs[k];
        L += f * ls[k];
    }
    const int r = row0 + rr;
    const int h = kvh * p.g + r / p.M, m = r % p.M;
    const int64_t row = (int64_t)(b * p.Hq + h) * p.M + m;
    if (p.out_bf16) {
        const u2 ov = {(uint32_t)f32_to_bf16_rne(o[0] / L) | ((uint32_t)f32_to_bf16_rne(o[1] / L) << 16),
                       (uint32_t)f32_to_bf16_rne(o[2] / L) | ((uint32_t)f32_to_bf16_rne(o[3] / L) << 16)};
        *(u2 *)(p.out + row * D + 4 * q) = ov;
    } else {
        const h4 ov = {(_Float16)(o[0] / L), (_Float16)(o[1] / L), (_Float16)(o[2] / L), (_Float16)(o[3] / L)};
        *(h4 *)(p.out + row * D + 4 * q) = ov;
    }
    if (q == 0 && p.rowstats) {
        p.rowstats[2 * row] = M;
        p.rowstats[2 * row + 1] = 1.0f / (L * (1.0f / 128.0f));  // 1 / L, the 2^7 probability scale undone
    }
}

template <int D>
__global__ __launch_bounds__(256) void decode_reduce_kernel(const DecodeParams p) {
    __shared__ float sm[256 / (D / 4)], sls[256 / (D / 4)];
    __shared__ f4 accl[256 / (D / 4)][D / 4];
    merge_split_row<D>(p, blockIdx.x, blockIdx.y, sm, sls, accl);
}

// Normalise the stashed logits into attention weights, 2^(x sl2 - M) / L, and/or
// accumulate the importance EMA.  Workgroup = 64 tokens x 16 row lanes: thread
// (token t, row lane rl) walks rows rl, rl+16, ... for tokens t, t+16, t+32,
// t+48; the row lanes are summed through LDS.
__global__ __launch_bounds__(256) void weights_importance_kernel(const DecodeParams p) {
    __shared__ float red[16][65];
    const float sl2 = p.scale_log2;
    const int64_t rows = (int64_t)p.B * p.Hq * p.M;
    const int t = threadIdx.x & 15, rl = threadIdx.x >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * 64 + t;
    float imp[4] = {0.f, 0.f, 0.f, 0.f};
    const int64_t N = p.N;
    for (int64_t r = rl; r < rows; r += 16) {
        const float M = p.rowstats[2 * r], inv = p.rowstats[2 * r + 1];
        float *srow = p.stash + r * N;
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = (n0 + 16 * i < N) ? srow[n0 + 16 * i] : -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float e = (M == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(__builtin_fmaf(x[i], sl2, -M));
            const float wgt = e * inv;
            if (p.attn_out && n0 + 16 * i < N) srow[n0 + 16 * i] = wgt;
            imp[i] += (n0 + 16 * i < N) ? wgt : 0.f;
        }
    }
    if (!p.scores) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) red[rl][16 * i + t] = imp[i];
    __syncthreads();
    if (threadIdx.x < 64) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) s += red[k][threadIdx.x];
        const int64_t n = (int64_t)blockIdx.x * 64 + threadIdx.x;
        if (n < p.n_scores) {
            // mean over (batch, head), summed over query positions
            float sc = p.scores[n] * p.decay;
            sc = sc + s / (float)(p.B * p.Hq);
            p.scores[n] = sc;
        }
    }
}

// Attention weights and importance EMA from the logit stash and the row
// statistics written by the fast kernel's in-kernel split merge.  Workgroup =
// 4 * kWsQuads tokens; thread (token quad q, row lane rl) reads 4 consecutive
// tokens of every (256 / kWsQuads)-th row (16-byte loads when the rows are
// 16-byte aligned); the row statistics and the old score come with the same
// batch of loads.
#ifndef AKV_WS_QUADS
#define AKV_WS_QUADS 8
#endif
// token quads per workgroup (4 tokens each): 8 (32 tokens, 32 row lanes) measured
// fastest at the 32k workload (16: +0.6 us per layer, 4: +2.5 us, 32: +13 us)
constexpr int kWsQuads = AKV_WS_QUADS;
// RB: rows per thread and batch of loads, chosen by the host so that one batch covers
// every row when there are few (the 32k Qwen layer: 96 rows, 3 per thread), else 8.
template <bool VEC, int RB>
__global__ __launch_bounds__(256) void weights_stats_kernel(const DecodeParams p) {
    constexpr int NQ = kWsQuads, TPW = 4 * NQ, NRL = 256 / NQ;  // tokens per workgroup, row lanes
    __shared__ float red[NRL][TPW + 1];
    const int tid = threadIdx.x, q = tid % NQ, rl = tid / NQ;
    const int64_t rows = (int64_t)p.B * p.Hq * p.M, N = p.N;
    const float sl2 = p.scale_log2;
    const int64_t n0 = (int64_t)blockIdx.x * TPW + 4 * q;
    // the old score is loaded with the first batch of logits, not after the reduction
    const int64_t ns = (int64_t)blockIdx.x * TPW + tid;
    const float sc_old = (p.scores && tid < TPW && ns < p.n_scores) ? p.scores[ns] : 0.f;
    float imp[4] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t r0 = rl; r0 < rows; r0 += NRL * RB) {
        f4 x[RB];
        float M[RB], W[RB];
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int64_t r = r0 + NRL * j;
            M[j] = -INFINITY;
            W[j] = 0.f;
            x[j] = (f4){-INFINITY, -INFINITY, -INFINITY, -INFINITY};
            if (r < rows) {
                M[j] = p.rowstats[2 * r];
                W[j] = p.rowstats[2 * r + 1];
                const float *src = p.stash + r * N + n0;
                if (VEC && n0 + 3 < N) {
                    x[j] = __builtin_nontemporal_load((const f4 *)src);  // read once
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (n0 + i < N) x[j][i] = src[i];
                }
            }
        }
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int64_t r = r0 + NRL * j;
            if (r >= rows) break;
            f4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = (M[j] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(__builtin_fmaf(x[j][i], sl2, -M[j]));
                w[i] = e * W[j];
                if (n0 + i < N) imp[i] += w[i];
            }
            if (p.attn_out) {
                float *dst = p.stash + r * N + n0;
                if (VEC && n0 + 3 < N) {
                    *(f4 *)dst = w;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (n0 + i < N) dst[i] = w[i];
                }
            }
        }
    }
    if (!p.scores) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) red[rl][4 * q + i] = imp[i];
    __syncthreads();
    if (tid < TPW) {
        float sacc = 0.f;
#pragma unroll
        for (int k = 0; k < NRL; ++k) sacc += red[k][tid];
        if (ns < p.n_scores) {
            // mean over (batch, head), summed over query positions
            float sc = sc_old * p.decay;
            sc = sc + sacc / (float)(p.B * p.Hq);
            p.scores[ns] = sc;
        }
    }
}

// Split merge + attention weights / importance EMA in one launch (the stash
// path).  Every workgroup first rebuilds the statistics of every query row
// from the split partials -- M = max_s m_s, L = sum_s 2^(m_s - M) l_s (x 2^7)
// -- into LDS; workgroup i < B*Hkv*nchunk*prows also merges the output of one
// row (as decode_reduce_kernel); then each workgroup normalises 64 tokens of
// every row, w = 2^(s - M) * 128 / L, writes them when the weights are asked
// for and adds sum_rows w / (B*Hq) to the importance EMA.  Loads of a phase
// are issued together.  Needs rows <= kFinishRows.
constexpr int kFinishRows = 1024;

template <int D>
__global__ __launch_bounds__(256) void finish_kernel(const DecodeParams p) {
    __shared__ float sm[256 / (D / 4)], sls[256 / (D / 4)];
    __shared__ f4 accl[256 / (D / 4)][D / 4];
    __shared__ float rM[kFinishRows], rW[kFinishRows];
    __shared__ float red[16][65];
    const int tid = threadIdx.x;
    const int rows = p.B * p.Hq * p.M;
    const int ns = p.nsplit;
    const float sl2 = p.scale_log2;
    const int64_t PS = D + 4;
    const int64_t pstride = (int64_t)p.prows * PS;

    // output merge of one (chunk, row), unless the split kernel merged its own splits
    const int n_merge = p.split_ctr ? 0 : p.B * p.Hkv * p.nchunk * p.prows;
    if ((int)blockIdx.x < n_merge)
        merge_split_row<D>(p, blockIdx.x / p.prows, blockIdx.x % p.prows, sm, sls, accl);

    // statistics of every row: from the split kernel's merge, or one thread per
    // row with all its split loads in flight
    if (p.split_ctr) {
        for (int r = tid; r < rows; r += 256) {
            rM[r] = p.rowstats[2 * r];
            rW[r] = p.rowstats[2 * r + 1];
        }
    }
    for (int r = tid; r < rows && !p.split_ctr; r += 256) {
        const int b = r / (p.Hq * p.M), hm = r % (p.Hq * p.M);
        const int h = hm / p.M, m = hm % p.M;
        const int kvh = h / p.g, rk = (h % p.g) * p.M + m;  // row within the kv-head's g*M rows
        const float *pp = p.part + ((int64_t)(b * p.Hkv + kvh) * p.nchunk + rk / 16) * ns * pstride + (rk % 16) * PS;
        float M = -INFINITY, L = 0.f;
        for (int s0 = 0; s0 < ns; s0 += 16) {
            float ms[16], ls[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                ms[k] = s0 + k < ns ? pp[(int64_t)(s0 + k) * pstride] : -INFINITY;
                ls[k] = s0 + k < ns ? pp[(int64_t)(s0 + k) * pstride + 1] : 0.f;
            }
            float nm = M;
#pragma unroll
            for (int k = 0; k < 16; ++k) nm = fmaxf(nm, ms[k]);
            if (nm == -INFINITY) continue;
            L *= (M == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(M - nm);
#pragma unroll
            for (int k = 0; k < 16; ++k) L += (ms[k] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ms[k] - nm) * ls[k];
            M = nm;
        }
        rM[r] = M;
        rW[r] = 128.0f / L;  // undo the 2^7 probability scale
    }
    __syncthreads();

    // weights and importance of tokens 64*blockIdx.x .. +63
    const int64_t N = p.N;
    const int64_t nmax = N > p.n_scores ? N : p.n_scores;
    if ((int64_t)blockIdx.x * 64 >= nmax) return;
    const int t = tid & 15, rl = tid >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * 64 + t;
    float imp[4] = {0.f, 0.f, 0.f, 0.f};
    constexpr int RB = 8;  // rows per batch of loads
    for (int r0 = rl; r0 < rows; r0 += 16 * RB) {
        float x[RB][4];
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int r = r0 + 16 * j;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                x[j][i] = (r < rows && n0 + 16 * i < N) ? p.stash[(int64_t)r * N + n0 + 16 * i] : -INFINITY;
        }
#pragma unroll
        for (int j = 0; j < RB; ++j) {
            const int r = r0 + 16 * j;
            if (r >= rows) break;
            const float M = rM[r], W = rW[r];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = (M == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(__builtin_fmaf(x[j][i], sl2, -M));
                const float wgt = e * W;
                if (n0 + 16 * i < N) {
                    if (p.attn_out) p.stash[(int64_t)r * N + n0 + 16 * i] = wgt;
                    imp[i] += wgt;
                }
            }
        }
    }
    if (!p.scores) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) red[rl][16 * i + t] = imp[i];
    __syncthreads();
    if (tid < 64) {
        float sacc = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) sacc += red[k][tid];
        const int64_t n = (int64_t)blockIdx.x * 64 + tid;
        if (n < p.n_scores) {
            // mean over (batch, head), summed over query positions
            float sc = p.scores[n] * p.decay;
            sc = sc + sacc / (float)(p.B * p.Hq);
            p.scores[n] = sc;
        }
    }
}

// Legacy symmetric-branch detection: flag[i] = 1 iff every zero-point of K (i=0) / V (i=1) is 0.
__global__ __launch_bounds__(1024) void legacy_sym_kernel(const void *kz, const void *vz, int64_t n, int dt,
                                                         int *flags) {
    __shared__ int any[2];
    if (threadIdx.x < 2) any[threadIdx.x] = 0;
    __syncthreads();
    int nzk = 0, nzv = 0;
    for (int64_t i = threadIdx.x; i < n; i += 1024) {
        nzk |= load_as_f32(kz, i, dt) != 0.0f;
        nzv |= load_as_f32(vz, i, dt) != 0.0f;
    }
    if (nzk) atomicOr(&any[0], 1);
    if (nzv) atomicOr(&any[1], 1);
    __syncthreads();
    if (threadIdx.x == 0) {
        flags[0] = any[0] ? 0 : 1;
        flags[1] = any[1] ? 0 : 1;
    }
}

// ------------------------------------------------------------------ launch

template <int D, int KB, int VB, int WK>
static hipError_t launch_split(const DecodeParams &p, hipStream_t stream) {
    dim3 grid(p.nsplit, p.Hkv, p.B * p.nchunk);
    const size_t lds_stage = kNW * 2816;
    const size_t lds_merge = (size_t)(2 * kNW * 16 + kNW * 16 * D) * 4;
    const size_t lds = lds_stage > lds_merge ? lds_stage : lds_merge;
    if (WK == AKV_WARM_AFFINE && p.n_out > 0)
        hipLaunchKernelGGL((decode_split_kernel<D, KB, VB, WK, WK == AKV_WARM_AFFINE>), grid, dim3(256), lds, stream, p);
    else
        hipLaunchKernelGGL((decode_split_kernel<D, KB, VB, WK, false>), grid, dim3(256), lds, stream, p);
    return hipGetLastError();
}

template <int D>
static hipError_t launch_split_bits(const DecodeParams &p, int kb, int vb, int wk, hipStream_t s) {
    if (wk == AKV_WARM_LEGACY) {
        if (kb == 2 && vb == 2) return launch_split<D, 2, 2, AKV_WARM_LEGACY>(p, s);
        if (kb == 4 && vb == 4) return launch_split<D, 4, 4, AKV_WARM_LEGACY>(p, s);
        if (kb == 8 && vb == 8) return launch_split<D, 8, 8, AKV_WARM_LEGACY>(p, s);
        return hipErrorInvalidValue;
    }
#define AKV_KV(a, b) \
    if (kb == a && vb == b) return launch_split<D, a, b, AKV_WARM_AFFINE>(p, s);
    AKV_KV(2, 2) AKV_KV(2, 3) AKV_KV(2, 4) AKV_KV(3, 2) AKV_KV(3, 3) AKV_KV(3, 4) AKV_KV(4, 2) AKV_KV(4, 3)
    AKV_KV(4, 4)
#undef AKV_KV
    return hipErrorInvalidValue;
}

hipError_t legacy_sym_launch(const void *kz, const void *vz, int64_t n, int dt, int *flags, hipStream_t s) {
    hipLaunchKernelGGL(legacy_sym_kernel, dim3(1), dim3(1024), 0, s, kz, vz, n, dt, flags);
    return hipGetLastError();
}

hipError_t decode_reduce_launch(const DecodeParams &p, hipStream_t s) {
    if (p.nsplit <= 8) {
        const int rpw = 256 / (p.D / 4);
        const dim3 g(p.B * p.Hkv * p.nchunk, (p.prows + rpw - 1) / rpw);
        if (p.D == 64) hipLaunchKernelGGL(reduce_few_kernel<64>, g, dim3(256), 0, s, p);
        else hipLaunchKernelGGL(reduce_few_kernel<128>, g, dim3(256), 0, s, p);
        return hipGetLastError();
    }
    const dim3 rgrid(p.B * p.Hkv * p.nchunk, p.prows);
    if (p.D == 64) hipLaunchKernelGGL(decode_reduce_kernel<64>, rgrid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(decode_reduce_kernel<128>, rgrid, dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t decode_launch(const DecodeParams &p, int kb, int vb, int wk, const int *sym_src_dt_n, hipStream_t s) {
    hipError_t e;
    if (wk == AKV_WARM_LEGACY && p.sym_flags && sym_src_dt_n) {
        e = legacy_sym_launch(p.kz, p.vz, (int64_t)sym_src_dt_n[1], sym_src_dt_n[0], (int *)p.sym_flags, s);
        if (e != hipSuccess) return e;
    }
    if (p.split_ctr && !decode_fast_eligible(p, wk)) return hipErrorInvalidValue;  // only the fast kernel merges
    if (decode_fast_eligible(p, wk)) e = decode_fast_split_launch(p, kb, vb, wk, s);
    else e = (p.D == 64) ? launch_split_bits<64>(p, kb, vb, wk, s) : launch_split_bits<128>(p, kb, vb, wk, s);
    if (e != hipSuccess) return e;
    const int64_t rows = (int64_t)p.B * p.Hq * p.M;
    if (p.stash && p.split_ctr) {
        // the split kernel merged its splits and wrote the row statistics
        const int64_t nmax = p.N > p.n_scores ? p.N : p.n_scores;
        const dim3 g((unsigned)((nmax + 4 * kWsQuads - 1) / (4 * kWsQuads)));
        constexpr int NRL = 256 / kWsQuads;
        const int64_t per = (rows + NRL - 1) / NRL;  // rows per thread
#define AKV_WS(RB)                                                                                 \
    do {                                                                                           \
        if (p.N % 4 == 0) hipLaunchKernelGGL((weights_stats_kernel<true, RB>), g, dim3(256), 0, s, p); \
        else hipLaunchKernelGGL((weights_stats_kernel<false, RB>), g, dim3(256), 0, s, p);        \
    } while (0)
        if (per <= 1) AKV_WS(1);
        else if (per <= 2) AKV_WS(2);
        else if (per <= 3) AKV_WS(3);
        else if (per <= 4) AKV_WS(4);
        else AKV_WS(8);
#undef AKV_WS
        return hipGetLastError();
    }
    if (p.stash && rows <= kFinishRows) {
        // one launch: output merge (unless the split kernel did it) + weights / importance
        const int64_t nmax = p.N > p.n_scores ? p.N : p.n_scores;
        const int64_t n_tok = (nmax + 63) / 64, n_merge = p.split_ctr ? 0 : (int64_t)p.B * p.Hkv * p.nchunk * p.prows;
        const unsigned nwg = (unsigned)(n_tok > n_merge ? n_tok : n_merge);
        if (p.D == 64) hipLaunchKernelGGL(finish_kernel<64>, dim3(nwg), dim3(256), 0, s, p);
        else hipLaunchKernelGGL(finish_kernel<128>, dim3(nwg), dim3(256), 0, s, p);
        return hipGetLastError();
    }
    if (!p.split_ctr && (e = decode_reduce_launch(p, s)) != hipSuccess) return e;
    if (p.stash) {
        const int64_t nmax = p.N > p.n_scores ? p.N : p.n_scores;
        hipLaunchKernelGGL(weights_importance_kernel, dim3((unsigned)((nmax + 63) / 64)), dim3(256), 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace akv
