// Split-K fused dequant-attention over a hot fp16 + warm packed KV cache.
//
// Grid: (split, kv-head, batch * row-chunk).  A workgroup owns one
// (batch, kv-head) and one contiguous token range of either the warm or the
// hot segment.  Its query rows are the Hq/Hkv query heads (x M query
// positions) that share the kv head -- up to 16 rows, the N dimension of the
// matrix-core tiles, so every K/V byte loaded feeds all of them.
//
// Per 16-token tile a wave:
//   QK:  S^T[16 tok x 16 rows] = K_tile . Q^T  -- 16x16x32 f16 MFMA; each lane
//        dequantizes the codes of one token for D/4 channels straight from
//        the packed row into the A operand (no LDS), K scale/zero pairs come
//        from a per-block LDS copy laid out in pair order.
//   softmax: online, log2 domain, lazy rescale (only when a row max grows by
//        more than 8); probabilities go to fp16 scaled by 2^7.
//   PV:  O^T[16 chunks x 16 rows] += V^T . P^T -- 16x16x16 f16 MFMA; the A
//        operand holds 4 tokens x 1 channel, so each lane reads one 8-channel
//        chunk of 4 tokens and builds (token, token) half pairs.
// Waves merge in LDS; one (m, l, acc) partial per workgroup goes to the
// workspace and akv_reduce_kernel merges the splits (log-sum-exp).
#include "akv_common.h"
#include "decode.h"

namespace akv {

constexpr int kThresh = 8;     // lazy-rescale threshold (log2 units)
constexpr float kPScale = 128.0f;  // fp16 probabilities carry a 2^7 factor

template <int D>
struct Geo {
    static constexpr int KSTEPS = D / 32;       // QK MFMA k-steps
    static constexpr int LCH = D / 4;           // K channels per lane group
    static constexpr int NPAIRS = LCH / 2;      // K code pairs per lane
    static constexpr int VCH = D / 8;           // 8-channel V chunks (MFMA rows used)
};

template <int BITS>
struct KRaw {  // raw K code dwords a lane holds for one token
    static constexpr int bytes(int lch) { return lch * BITS / 8; }
};

// LDS layout of one wave's staging area (bytes)
template <int D>
struct WaveLds {
    static constexpr int KMETA = 2 * 4 * (D / 8) * 4;  // [s|z][grp][pair] u32
    static constexpr int VMETA = 2 * 16 * 16 * 4;      // [s|z][group<=16][16 tokens] f32 or f16
    static constexpr int BYTES = KMETA + VMETA;
};

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

template <int D>
struct WaveState {
    float m;        // running max (log2 domain) of this lane's row
    float l;        // partial sum of exp2(s - m) over this lane's tokens
    f4 acc[8];      // O^T: acc[j][i] = chunk (4*grp+i), channel slot j, row col
};

// One tile's softmax + PV given S^T (this lane: tokens 4*grp+i, row col) and
// the V^T operands vop[j] (chunk col, tokens 4*grp..+3, channel slot j).
template <int D>
__device__ __forceinline__ void softmax_pv(WaveState<D> &st, f4 s, const h4 *vop) {
    float tmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    tmax = wave_max16(tmax);
    const bool need = tmax > st.m + (float)kThresh;
    if (__builtin_amdgcn_ballot_w64(need)) {  // wave-uniform
        const float mn = fmaxf(st.m, tmax);
        const float alpha = (mn == -INFINITY) ? 1.0f : exp2f(st.m - mn);
        st.l *= alpha;
#pragma unroll
        for (int j = 0; j < 8; ++j) st.acc[j] *= alpha;
        st.m = mn;
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = (st.m == -INFINITY) ? 0.0f : exp2f(s[i] - st.m);
    st.l += (p[0] + p[1]) + (p[2] + p[3]);
    h4 pop;
#pragma unroll
    for (int i = 0; i < 4; ++i) pop[i] = (_Float16)(p[i] * kPScale);
#pragma unroll
    for (int j = 0; j < 8; ++j) st.acc[j] = mfma_k16(vop[j], pop, st.acc[j]);
}

template <int D>
__device__ __forceinline__ void store_stash(const DecodeParams &p, int b, int row_valid, int h, int m,
                                            int64_t nlog0, const f4 &s, const bool *valid) {
    if (!p.stash || !row_valid) return;
    float *dst = p.stash + ((int64_t)(b * p.Hq + h) * p.M + m) * p.N + nlog0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (valid[i]) dst[i] = s[i];
}

template <int D, int KB, int VB, int WK>
__global__ __launch_bounds__(256) void decode_split_kernel(const DecodeParams p) {
    using G = Geo<D>;
    constexpr int NW = 4;
    constexpr int KSTEPS = G::KSTEPS, LCH = G::LCH, NPAIRS = G::NPAIRS, VCH = G::VCH;
    constexpr int KBYTES = LCH * KB / 8;       // warm K code bytes per lane
    constexpr int KDW = (KBYTES + 3) / 4;

    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int split = blockIdx.x, kvh = blockIdx.y;
    const int b = blockIdx.z / p.nchunk, chunk = blockIdx.z % p.nchunk;
    const int row0 = chunk * 16;
    const int nrows = min(16, p.R - row0);
    const bool is_warm = split < p.n_wsplit;

    // this lane's query row (as the N column of the MFMA tiles)
    const int r = row0 + col;
    const int row_valid = col < nrows;
    const int hq = kvh * p.g + (row_valid ? r / p.M : 0);
    const int mq = row_valid ? r % p.M : 0;

    // segment-local token range of this split
    int64_t t_begin, t_end;
    if (is_warm) {
        t_begin = (int64_t)split * p.wsplit_len;
        t_end = min(t_begin + p.wsplit_len, p.n_warm);
    } else {
        t_begin = (int64_t)(split - p.n_wsplit) * p.hsplit_len;
        t_end = min(t_begin + p.hsplit_len, p.n_hot);
    }
    // logical index of segment token 0
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
                int ch;
                if (!is_warm) ch = kpair_chan<16>(pi, hf);
                else ch = kpair_chan<KB>(pi, hf);
                qop[st][j] = row_valid ? qrow[ch] : (_Float16)0.0f;
            }
    }

    WaveState<D> stt;
    stt.m = -INFINITY;
    stt.l = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) stt.acc[j] = (f4){0.f, 0.f, 0.f, 0.f};

    unsigned char *wlds = smem + wave * WaveLds<D>::BYTES;
    uint32_t *kmeta_lds = (uint32_t *)wlds;                          // [2][4][NPAIRS]
    unsigned char *vmeta_lds = wlds + WaveLds<D>::KMETA;            // [2][ng][16]

    const int64_t bh = (int64_t)b * p.Hkv + kvh;
    const float sl2 = p.scale_log2;

    if (!is_warm) {
        // ------------------------------------------------------------ hot tiles
        const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.khot + bh * p.n_hot * D, (uint32_t)(p.n_hot * D * 2));
        const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.vhot + bh * p.n_hot * D, (uint32_t)(p.n_hot * D * 2));
        for (int64_t t0 = t_begin + 16 * wave; t0 < t_end; t0 += 16 * NW) {
            // K: lane's token t0+col, channels LCH*grp .. +LCH (fp16, natural order)
            const int64_t tk = t0 + col;
            h8 kop[KSTEPS];
#pragma unroll
            for (int st = 0; st < KSTEPS; ++st) {
                u4 raw = bld128(rk, (uint32_t)((tk * D + LCH * grp + 8 * st) * 2));
                kop[st] = __builtin_bit_cast(h8, raw);
            }
            f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < KSTEPS; ++st) s = mfma_k32(kop[st], qop[st], s);
            bool valid[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                valid[i] = (t0 + 4 * grp + i) < t_end;
                s[i] = valid[i] ? s[i] * sl2 : -INFINITY;
            }
            store_stash<D>(p, b, row_valid, hq, mq, seg_base + t0 + 4 * grp, s, valid);
            // V: lane's chunk col (8 channels), tokens t0+4*grp .. +3
            h4 vop[8];
            {
                u4 w[4];
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int64_t tv = t0 + 4 * grp + jj;
                    w[jj] = (col < VCH && tv < t_end) ? bld128(rv, (uint32_t)((tv * D + 8 * col) * 2))
                                                      : (u4){0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                    const uint32_t lo = perm(w[1][j / 2], w[0][j / 2], sel);
                    const uint32_t hi = perm(w[3][j / 2], w[2][j / 2], sel);
                    vop[j] = __builtin_bit_cast(h4, (u2){lo, hi});
                }
            }
            softmax_pv<D>(stt, s, vop);
        }
    } else {
        // ----------------------------------------------------------- warm tiles
        const int unit = (WK == AKV_WARM_AFFINE) ? p.T : 16;  // tokens sharing K meta
        const int64_t hw = (WK == AKV_WARM_AFFINE) ? bh : (p.warm_heads == 1 ? 0 : kvh);
        const __amdgpu_buffer_rsrc_t rkc =
            make_rsrc((const unsigned char *)p.kc + hw * p.n_warm * p.kc_row, (uint32_t)(p.n_warm * p.kc_row));
        const __amdgpu_buffer_rsrc_t rvc =
            make_rsrc((const unsigned char *)p.vc + hw * p.n_warm * p.vc_row, (uint32_t)(p.n_warm * p.vc_row));
        int ksym = 0, vsym = 0;
        if (WK == AKV_WARM_LEGACY) {
            ksym = p.sym_flags ? p.sym_flags[0] : p.legacy_sym;
            vsym = p.sym_flags ? p.sym_flags[1] : p.legacy_sym;
        }
        for (int64_t u0 = t_begin + (int64_t)unit * wave; u0 < t_end; u0 += (int64_t)unit * NW) {
            // ---- K meta for this unit -> LDS in pair order (affine: per channel of the block)
            if (WK == AKV_WARM_AFFINE) {
                const int64_t blk = u0 / p.T;
                const _Float16 *ks = (const _Float16 *)p.ks + (bh * p.nblk + blk) * D;
                const _Float16 *kz = (const _Float16 *)p.kz + (bh * p.nblk + blk) * D;
                // lane -> (grp' = lane/16, pair = lane%16); pairs >= NPAIRS unused for D=64
                const int g2 = lane >> 4, pi = lane & 15;
                if (pi < NPAIRS) {
                    int clo = 0, chi = 0;
#pragma unroll
                    for (int q = 0; q < NPAIRS; ++q)
                        if (q == pi) { clo = kpair_chan<KB>(q, 0); chi = kpair_chan<KB>(q, 1); }
                    const int base = LCH * g2;
                    h2 sv = {ks[base + clo], ks[base + chi]};
                    h2 zv = {kz[base + clo], kz[base + chi]};
                    kmeta_lds[(0 * 4 + g2) * NPAIRS + pi] = as_u32(sv);
                    kmeta_lds[(1 * 4 + g2) * NPAIRS + pi] = as_u32(zv);
                }
                __builtin_amdgcn_wave_barrier();
            }
            const int64_t u1 = min(u0 + unit, t_end);
            for (int64_t t0 = u0; t0 < u1; t0 += 16) {
                // ---- K codes: lane's token t0+col, channels LCH*grp..+LCH
                const int64_t tk = t0 + col;
                uint32_t kr[4] = {0u, 0u, 0u, 0u};
                uint32_t kr8[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
                {
                    const uint32_t off = (uint32_t)(tk * p.kc_row + KBYTES * grp);
                    if (KB == 8) {
#pragma unroll
                        for (int q = 0; q < KDW; q += 4) {
                            u4 x = bld128(rkc, off + 4 * q);
                            kr8[q] = x[0]; kr8[q + 1] = x[1]; kr8[q + 2] = x[2]; kr8[q + 3] = x[3];
                        }
                    } else if (KBYTES == 12) { u3 x = bld96(rkc, off); kr[0] = x[0]; kr[1] = x[1]; kr[2] = x[2]; }
                    else if (KBYTES == 16) { u4 x = bld128(rkc, off); kr[0] = x[0]; kr[1] = x[1]; kr[2] = x[2]; kr[3] = x[3]; }
                    else if (KBYTES == 8) { u2 x = bld64(rkc, off); kr[0] = x[0]; kr[1] = x[1]; }
                    else if (KBYTES == 6) {  // 3-bit, D=64: 6 bytes at a 2-byte-aligned offset
                        const uint32_t base = off & ~3u;
                        const int sh = (int)(off - base);
                        u3 x = bld96(rkc, base);
                        kr[0] = __builtin_amdgcn_alignbyte(x[1], x[0], sh);
                        kr[1] = __builtin_amdgcn_alignbyte(x[2], x[1], sh) & 0xFFFFu;
                    }
                    else if (KBYTES == 4) { kr[0] = bld32(rkc, off); }
                }
                // ---- K meta for this tile
                h2 ksc[NPAIRS], kze[NPAIRS];
                if (WK == AKV_WARM_AFFINE) {
#pragma unroll
                    for (int q = 0; q < NPAIRS; ++q) {
                        ksc[q] = as_h2(kmeta_lds[(0 * 4 + grp) * NPAIRS + q]);
                        kze[q] = as_h2(kmeta_lds[(1 * 4 + grp) * NPAIRS + q]);
                    }
                }
                float lks[4] = {0.f, 0.f, 0.f, 0.f}, lkz[4] = {0.f, 0.f, 0.f, 0.f};
                if (WK == AKV_WARM_LEGACY) {
                    // groups covering channels LCH*grp .. +LCH (gs >= 8, power of two)
                    const int ng = LCH / p.gs > 0 ? LCH / p.gs : 1;
                    const int64_t mrow = hw * p.n_warm + min(tk, p.n_warm - 1);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (q < ng) {
                            const int gi = (LCH * grp) / p.gs + q;
                            lks[q] = load_as_f32(p.ks, mrow * p.lg + gi, p.meta_dt);
                            lkz[q] = load_as_f32(p.kz, mrow * p.lg + gi, p.meta_dt);
                        }
                }
                // ---- dequant + QK
                f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < KSTEPS; ++st) {
                    h8 a;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int pi = 4 * st + k;
                        const uint32_t cp = (KB == 8) ? kpair_extract<8>(kr8, pi) : kpair_extract<KB>(kr, pi);
                        h2 v;
                        if (WK == AKV_WARM_AFFINE) {
                            v = deq_affine(cp, ksc[pi], kze[pi]);
                        } else {
                            const int c0 = kpair_chan<KB>(pi, 0), c1 = kpair_chan<KB>(pi, 1);
                            const int q0 = (LCH / p.gs > 0) ? c0 / p.gs : 0;
                            const int q1 = (LCH / p.gs > 0) ? c1 / p.gs : 0;
                            const float s0 = q0 == 0 ? lks[0] : q0 == 1 ? lks[1] : q0 == 2 ? lks[2] : lks[3];
                            const float s1 = q1 == 0 ? lks[0] : q1 == 1 ? lks[1] : q1 == 2 ? lks[2] : lks[3];
                            const float z0 = q0 == 0 ? lkz[0] : q0 == 1 ? lkz[1] : q0 == 2 ? lkz[2] : lkz[3];
                            const float z1 = q1 == 0 ? lkz[0] : q1 == 1 ? lkz[1] : q1 == 2 ? lkz[2] : lkz[3];
                            const float u0f = (float)(cp & 0xFFFFu), u1f = (float)(cp >> 16);
                            float d0, d1;
                            if (ksym) { d0 = (u0f - p.half_max_k) * s0; d1 = (u1f - p.half_max_k) * s1; }
                            else { d0 = u0f * s0; d0 = d0 + z0; d1 = u1f * s1; d1 = d1 + z1; }
                            v = (h2){(_Float16)d0, (_Float16)d1};
                        }
                        a[2 * k] = v[0];
                        a[2 * k + 1] = v[1];
                    }
                    s = mfma_k32(a, qop[st], s);
                }
                bool valid[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    valid[i] = (t0 + 4 * grp + i) < t_end;
                    s[i] = valid[i] ? s[i] * sl2 : -INFINITY;
                }
                // ---- K outlier channels (affine): replace the dequantized value of
                // channel d_j by the stored fp16 value -> add q[d_j]*(o - kdeq) to s
                if (WK == AKV_WARM_AFFINE && p.n_out > 0) {
                    const int64_t blk = t0 / p.T;
#pragma unroll 1
                    for (int j = 0; j < p.n_out; ++j) {
                        const int dj = min(max((int)p.k_oidx[((int64_t)b * p.nblk + blk) * p.n_out + j], 0), D - 1);
                        const float qd = row_valid ? (float)p.q[((int64_t)(b * p.Hq + hq) * p.M + mq) * D + dj] : 0.f;
                        const _Float16 ksj = ((const _Float16 *)p.ks)[(bh * p.nblk + blk) * D + dj];
                        const _Float16 kzj = ((const _Float16 *)p.kz)[(bh * p.nblk + blk) * D + dj];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            if (!valid[i]) continue;
                            const int64_t t = t0 + 4 * grp + i;
                            const unsigned char *row = (const unsigned char *)p.kc + (hw * p.n_warm + t) * p.kc_row;
                            const uint32_t code = extract_code(row, dj, KB);
                            const _Float16 kd = (_Float16)((_Float16)((_Float16)code * ksj) + kzj);
                            const _Float16 od = ((const _Float16 *)p.k_odata)[(bh * p.n_warm + t) * p.n_out + j];
                            s[i] += qd * ((float)od - (float)kd) * sl2;
                        }
                    }
                }
                store_stash<D>(p, b, row_valid, hq, mq, seg_base + t0 + 4 * grp, s, valid);

                // ---- V: lane's chunk col, tokens t0+4*grp .. +3
                uint32_t wv[4][2];
                {
                    constexpr int CB = VB;  // bytes per 8-channel chunk
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const int64_t tv = t0 + 4 * grp + jj;
                        wv[jj][0] = 0u; wv[jj][1] = 0u;
                        if (col < VCH) {
                            const uint32_t rowoff = (uint32_t)(tv * p.vc_row);
                            if (VB == 4) wv[jj][0] = bld32(rvc, rowoff + 4 * col);
                            else if (VB == 2) wv[jj][0] = bld16(rvc, rowoff + 2 * col);
                            else if (VB == 8) { u2 x = bld64(rvc, rowoff + 8 * col); wv[jj][0] = x[0]; wv[jj][1] = x[1]; }
                            else {  // 3-bit: 3 bytes at 3*col, read the aligned 8 bytes around them
                                const int off = (3 * col) & ~3;
                                const int sh = 3 * col - off;
                                u2 x = bld64(rvc, rowoff + off);
                                wv[jj][0] = __builtin_amdgcn_alignbyte(x[1], x[0], sh);
                            }
                        }
                        (void)CB;
                    }
                }
                // V meta: per token of the tile, for the group of chunk col -> LDS [s|z][group][token]
                h2 vs01 = {}, vs23 = {}, vz01 = {}, vz23 = {};
                float fvs[4] = {0.f, 0.f, 0.f, 0.f}, fvz[4] = {0.f, 0.f, 0.f, 0.f};
                {
                    const int ngr = (WK == AKV_WARM_AFFINE) ? D / p.Gv : p.lg;
                    const int tot = 16 * ngr;  // <= 16*16
                    for (int e = lane; e < tot; e += 64) {
                        const int tt = e / ngr, gg = e % ngr;
                        const int64_t tv = min(t0 + tt, p.n_warm - 1);
                        if (WK == AKV_WARM_AFFINE) {
                            const int64_t mi = (bh * p.n_warm + tv) * ngr + gg;
                            ((_Float16 *)vmeta_lds)[(0 * 16 + gg) * 16 + tt] = ((const _Float16 *)p.vs)[mi];
                            ((_Float16 *)vmeta_lds)[(1 * 16 + gg) * 16 + tt] = ((const _Float16 *)p.vz)[mi];
                        } else {
                            const int64_t mi = (hw * p.n_warm + tv) * ngr + gg;
                            ((float *)vmeta_lds)[(0 * 16 + gg) * 16 + tt] = load_as_f32(p.vs, mi, p.meta_dt);
                            ((float *)vmeta_lds)[(1 * 16 + gg) * 16 + tt] = load_as_f32(p.vz, mi, p.meta_dt);
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
                    const int gsz = (WK == AKV_WARM_AFFINE) ? p.Gv : p.gs;
                    const int gme = min((8 * col) / gsz, 15);
                    if (WK == AKV_WARM_AFFINE) {
                        const uint32_t *sp = (const uint32_t *)vmeta_lds + ((0 * 16 + gme) * 16 + 4 * grp) / 2;
                        const uint32_t *zp = (const uint32_t *)vmeta_lds + ((1 * 16 + gme) * 16 + 4 * grp) / 2;
                        vs01 = as_h2(sp[0]); vs23 = as_h2(sp[1]);
                        vz01 = as_h2(zp[0]); vz23 = as_h2(zp[1]);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            fvs[i] = ((const float *)vmeta_lds)[(0 * 16 + gme) * 16 + 4 * grp + i];
                            fvz[i] = ((const float *)vmeta_lds)[(1 * 16 + gme) * 16 + 4 * grp + i];
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
                }
                h4 vop[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t c01 = vpair_extract<VB>(wv[0], wv[1], j);
                    const uint32_t c23 = vpair_extract<VB>(wv[2], wv[3], j);
                    h2 a01, a23;
                    if (WK == AKV_WARM_AFFINE) {
                        a01 = deq_affine(c01, vs01, vz01);
                        a23 = deq_affine(c23, vs23, vz23);
                    } else {
                        float d[4];
                        const float u[4] = {(float)(c01 & 0xFFFFu), (float)(c01 >> 16), (float)(c23 & 0xFFFFu),
                                            (float)(c23 >> 16)};
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            if (vsym) d[i] = (u[i] - p.half_max_v) * fvs[i];
                            else { d[i] = u[i] * fvs[i]; d[i] = d[i] + fvz[i]; }
                        }
                        a01 = (h2){(_Float16)d[0], (_Float16)d[1]};
                        a23 = (h2){(_Float16)d[2], (_Float16)d[3]};
                    }
                    vop[j] = (h4){a01[0], a01[1], a23[0], a23[1]};
                }
                // V outliers: the chunk holding d_j gets the stored value (replace)
                if (WK == AKV_WARM_AFFINE && p.n_out > 0) {
                    const int64_t blk = t0 / p.T;
#pragma unroll 1
                    for (int j = 0; j < p.n_out; ++j) {
                        const int dj = min(max((int)p.v_oidx[((int64_t)b * p.nblk + blk) * p.n_out + j], 0), D - 1);
                        if (dj / 8 != col) continue;
                        const int within = dj % 8;
#pragma unroll
                        for (int jj = 0; jj < 8; ++jj) {
                            if (vpair_chan<VB>(jj) != within) continue;
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const int64_t tv = min(t0 + 4 * grp + i, p.n_warm - 1);
                                vop[jj][i] = ((const _Float16 *)p.v_odata)[(bh * p.n_warm + tv) * p.n_out + j];
                            }
                        }
                    }
                }
                softmax_pv<D>(stt, s, vop);
            }
        }
    }

    // ---- merge the waves of this workgroup, write the split partial
    stt.l = wave_sum16(stt.l);
    __syncthreads();
    float *mlds = (float *)smem;                   // [NW][16] max
    float *llds = mlds + NW * 16;                  // [NW][16] sum
    float *alds = llds + NW * 16;                  // [NW][16][D] acc
    if (grp == 0) {
        mlds[wave * 16 + col] = stt.m;
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
    float *part = p.part + ((bh * p.nchunk + chunk) * p.nsplit + split) * (int64_t)(p.prows * (D + 2));
    for (int e = threadIdx.x; e < nrows * D; e += 256) {
        const int rr = e / D, ch = e % D;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) mx = fmaxf(mx, mlds[w * 16 + rr]);
        float a = 0.f, l = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = mlds[w * 16 + rr];
            const float f = (mw == -INFINITY) ? 0.f : exp2f(mw - mx);
            a += f * alds[(w * 16 + rr) * D + ch];
            l += f * llds[w * 16 + rr];
        }
        part[rr * (D + 2) + 2 + ch] = a;
        if (ch == 0) {
            part[rr * (D + 2) + 0] = mx;
            part[rr * (D + 2) + 1] = l;
        }
    }
}

// Merge the split partials of one (batch, kv-head, row chunk): out = sum f_s acc_s / (L * 2^7),
// f_s = exp2(m_s - M); also records (M, L) per query row for the weights / importance pass.
template <int D>
__global__ __launch_bounds__(256) void decode_reduce_kernel(const DecodeParams p) {
    __shared__ float fac[16 * 256];
    __shared__ float rowM[16], rowL[16];
    const int bhc = blockIdx.x;
    const int chunk = bhc % p.nchunk;
    const int64_t bh = bhc / p.nchunk;
    const int b = (int)(bh / p.Hkv), kvh = (int)(bh % p.Hkv);
    const int row0 = chunk * 16, nrows = min(16, p.R - row0);
    const int ns = p.nsplit;
    const int64_t pstride = (int64_t)p.prows * (D + 2);
    const float *part = p.part + (bh * p.nchunk + chunk) * (int64_t)ns * pstride;
    if (threadIdx.x < nrows) {
        const int rr = threadIdx.x;
        float mx = -INFINITY;
        for (int s = 0; s < ns; ++s) mx = fmaxf(mx, part[s * pstride + rr * (D + 2)]);
        float l = 0.f;
        for (int s = 0; s < ns; ++s) {
            const float ms = part[s * pstride + rr * (D + 2)];
            const float f = (ms == -INFINITY) ? 0.f : exp2f(ms - mx);
            l += f * part[s * pstride + rr * (D + 2) + 1];
        }
        rowM[rr] = mx;
        rowL[rr] = l;
    }
    __syncthreads();
    const bool fit = ns <= 256;
    if (fit) {
        for (int e = threadIdx.x; e < nrows * ns; e += 256) {
            const int rr = e / ns, s = e % ns;
            const float ms = part[s * pstride + rr * (D + 2)];
            fac[rr * 256 + s] = (ms == -INFINITY) ? 0.f : exp2f(ms - rowM[rr]);
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < nrows * D; e += 256) {
        const int rr = e / D, ch = e % D;
        float a = 0.f;
        for (int s = 0; s < ns; ++s) {
            float f;
            if (fit) f = fac[rr * 256 + s];
            else {
                const float ms = part[s * pstride + rr * (D + 2)];
                f = (ms == -INFINITY) ? 0.f : exp2f(ms - rowM[rr]);
            }
            a += f * part[s * pstride + rr * (D + 2) + 2 + ch];
        }
        const float o = a / (rowL[rr] * kPScale);
        const int r = row0 + rr;
        const int h = kvh * p.g + r / p.M, m = r % p.M;
        p.out[((int64_t)(b * p.Hq + h) * p.M + m) * D + ch] = (_Float16)o;
    }
    if (threadIdx.x < nrows && p.rowstats) {
        const int r = row0 + threadIdx.x;
        const int h = kvh * p.g + r / p.M, m = r % p.M;
        const int64_t row = (int64_t)(b * p.Hq + h) * p.M + m;
        p.rowstats[2 * row] = rowM[threadIdx.x];
        p.rowstats[2 * row + 1] = rowL[threadIdx.x];
    }
}

// Normalise the stashed log2-domain logits into attention weights and/or
// accumulate the importance EMA.  One thread per token.
__global__ __launch_bounds__(256) void weights_importance_kernel(const DecodeParams p) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t rows = (int64_t)p.B * p.Hq * p.M;
    const int64_t nmax = max(p.N, p.n_scores);
    if (n >= nmax) return;
    float imp = 0.f;
    if (n < p.N) {
        for (int64_t row = 0; row < rows; ++row) {
            const float M = p.rowstats[2 * row], L = p.rowstats[2 * row + 1];
            const float s = p.stash[row * p.N + n];
            const float e = (M == -INFINITY) ? 0.f : exp2f(s - M);
            const float w = e / L;
            if (p.attn_out) p.attn_out[row * p.N + n] = w;
            imp += w;
        }
    }
    if (p.scores && n < p.n_scores) {
        // mean over (batch, head), summed over query positions
        const float mean = imp / (float)(p.B * p.Hq);
        float sc = p.scores[n] * p.decay;
        sc = sc + mean;
        p.scores[n] = sc;
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
    const size_t lds_stage = 4 * WaveLds<D>::BYTES;
    const size_t lds_merge = (size_t)(2 * 4 * 16 + 4 * 16 * D) * 4;
    const size_t lds = lds_stage > lds_merge ? lds_stage : lds_merge;
    hipLaunchKernelGGL((decode_split_kernel<D, KB, VB, WK>), grid, dim3(256), lds, stream, p);
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

hipError_t decode_launch(const DecodeParams &p, int kb, int vb, int wk, const int *sym_src_dt_n, hipStream_t s) {
    hipError_t e;
    if (wk == AKV_WARM_LEGACY && p.sym_flags && sym_src_dt_n) {
        e = legacy_sym_launch(p.kz, p.vz, (int64_t)sym_src_dt_n[1], sym_src_dt_n[0], (int *)p.sym_flags, s);
        if (e != hipSuccess) return e;
    }
    e = (p.D == 64) ? launch_split_bits<64>(p, kb, vb, wk, s) : launch_split_bits<128>(p, kb, vb, wk, s);
    if (e != hipSuccess) return e;
    if (p.D == 64) hipLaunchKernelGGL(decode_reduce_kernel<64>, dim3(p.B * p.Hkv * p.nchunk), dim3(256), 0, s, p);
    else hipLaunchKernelGGL(decode_reduce_kernel<128>, dim3(p.B * p.Hkv * p.nchunk), dim3(256), 0, s, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (p.stash) {
        const int64_t nmax = p.N > p.n_scores ? p.N : p.n_scores;
        hipLaunchKernelGGL(weights_importance_kernel, dim3((unsigned)((nmax + 255) / 256)), dim3(256), 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace akv
