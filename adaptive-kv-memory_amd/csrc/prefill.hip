// Chunked-prefill attention over a hot fp16 + block-affine warm KV cache:
// M query positions per head (a prompt chunk placed after every cached token,
// so no mask over the cache) against Nh + Nw cached tokens.  MFMA-bound.
//
// Workgroup: 8 waves, 256 query rows of one (batch, kv-head) -- row r is
// query head kvh*g + r / M at position r % M, so the g heads of a GQA group
// share every dequantized tile.  Wave w owns rows 32w .. 32w+31 as two
// 16-row MFMA column groups.
//
// The cache is walked in 32-token tiles (hot tiles, then warm units, then --
// when the chunk's own K/V are given -- the chunk's tokens under a causal mask:
// query position m sees chunk tokens 0..m), double buffered in LDS.  While the MFMAs consume tile j, waves 0-3 dequantize tile
// j+1's K and waves 4-7 its V from registers loaded one tile ahead:
//   K tile  [32 tokens][4 channel groups][16 code pairs] u32, pair order of
//           kpair_chan() (the query operand is permuted to match), exact
//           fp16 dequant round16(round16(c*s) + z) as in the decode kernel;
//   V tile  the PV MFMA operand, [channel kk of the chunk][half][token pair
//           of the lane's quad][lane] u32 (each staging wave writes 64
//           consecutive dwords; a reading lane takes its four dwords at a
//           256-byte stride), values round16(c*s); the zero-points enter
//           through one more MFMA with the tile's zeros [half][pair][lane]
//           (sum_t P z, added to every channel of the group).
// Per column group: S^T = K . Q^T for each 16-token half (4 x 16x16x32),
// online softmax over the 32 tokens in the log2 domain (P in fp16 x 2^7),
// O^T += V^T . P^T over the 32 tokens (8 x 16x16x32 + 1 for the zeros, whose
// last chunk row takes ones: the row sums of P come out of the same MFMA).
//
// Grid: one workgroup per (batch, kv-head, token split, row tile), the
// (batch, kv-head) index varying fastest so that consecutive workgroups --
// placed round-robin on the XCDs -- keep one kv-head's tiles in one L2.
// With one split the output is written directly; with more, the partials
// (m, l, acc) go to the decode split layout and decode_reduce_kernel merges.
#include "akv_common.h"
#include "decode.h"
#include "prefill.h"
#include "tile_common.h"

namespace akv {

namespace {

constexpr int kPD = 128;
constexpr int kPTok = 32;                      // tokens per tile
constexpr int kPThreads = 512;                 // 8 waves, 32 query rows each
constexpr int kKRow = 256 + 16;                // K tile row bytes (padded against bank conflicts)
constexpr int kKTile = kPTok * kKRow;          // 8704
constexpr int kVTile = 2 * 8 * 64 * 8;         // 8192
constexpr int kVzTile = 2 * 64 * 8;            // 1024
constexpr int kBuf = kKTile + kVTile + kVzTile;
constexpr int kPKmeta = 3 * 4 * 16 * 4;        // [s | n | z][group][pair] u32, per K wave
constexpr int kPLds = 2 * kBuf + 4 * kPKmeta;
constexpr uint32_t kOnes2 = 0x3C003C00u;       // fp16 pair (1, 1)

// bf16 pair (one dword) -> fp16 pair (exact for values in fp16's normal range)
__device__ __forceinline__ uint32_t bf16x2_to_h2(uint32_t w) {
    const h2 v = {(_Float16)bf16_to_f32((uint16_t)w), (_Float16)bf16_to_f32((uint16_t)(w >> 16))};
    return as_u32(v);
}

}  // namespace

// OWN: the chunk's own keys / values follow the cache (a variant of its own, so that the
// cache loop of the plain kernel keeps its registers)
template <int BK, int BV, int NG, bool OWN>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_kernel(const PrefillParams p) {
    constexpr int KR = 16 * BK, VR = 16 * BV, GV = kPD / NG;
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, grp = lane >> 4;

    // ---- workgroup -> (batch, kv-head, split, row tile); (b, kv-head) fastest
    const int npair = p.B * p.Hkv;
    const int id = blockIdx.x;
    const int pair = id % npair;
    const int rest = id / npair;
    const int split = rest % p.nsplit;
    const int rtile = rest / p.nsplit;
    const int b = pair / p.Hkv, kvh = pair % p.Hkv;
    const int64_t bh = (int64_t)b * p.Hkv + kvh;
    const int r0 = rtile * kPrefillRows;

    // ---- token tiles of this split: hot tiles first, then warm units, then the chunk's own
    const int n_ht = (int)((p.n_hot + kPTok - 1) / kPTok), n_wt = (int)((p.n_warm + kPTok - 1) / kPTok);
    const int c_first = n_ht + n_wt;  // first tile of the chunk's own tokens
    const int nt = c_first + (OWN ? (p.n_cur + kPTok - 1) / kPTok : 0);
    const int t_begin = (int)min((int64_t)split * p.tiles_per_split, (int64_t)nt);
    const int t_end = (int)min((int64_t)t_begin + p.tiles_per_split, (int64_t)nt);
    const int n_hot32 = (int)p.n_hot, n_warm32 = (int)p.n_warm;

    // ---- query operand of the wave's two column groups (rows past R repeat row r0)
    const float sl2 = p.scale_log2;
    h8 qop[2][4];
#pragma unroll
    for (int rg = 0; rg < 2; ++rg) {
        const int r = r0 + 32 * wave + 16 * rg + col;
        const int rc = r < p.R ? r : r0;
        const int hq = kvh * p.g + rc / p.M, mq = rc % p.M;
        const int64_t qoff = ((int64_t)(b * p.Hq + hq) * p.M + mq) * kPD + 32 * grp;
        const u4 *src = (const u4 *)((const uint16_t *)p.q + qoff);
        uint32_t nat[16], pairs[16];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const u4 x = src[q4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t xe = x[e];
                nat[4 * q4 + e] = p.q_bf16 ? bf16x2_to_h2(xe) : xe;
            }
        }
        hot_k_pairs<BK>(nat, pairs);
#pragma unroll
        for (int st = 0; st < 4; ++st)
            qop[rg][st] = __builtin_bit_cast(h8, (u4){pairs[4 * st], pairs[4 * st + 1], pairs[4 * st + 2], pairs[4 * st + 3]});
    }

    // With the chunk's own tokens a split that begins past the chunk's first tile can hold
    // no token a row sees (all masked): a finite start for the running max keeps such a
    // row's bias finite, so its probabilities are exp2(-inf) = 0 and its partial is
    // (max -2^126, sum 0), which the merge weights by exp2(-2^126 - max) = 0.
    Soft sm[2];
#pragma unroll
    for (int rg = 0; rg < 2; ++rg) {
        sm[rg].m2 = OWN ? -0x1p126f : -INFINITY;
        sm[rg].l = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) sm[rg].acc[j] = (f4){0.f, 0.f, 0.f, 0.f};
        sm[rg].accz = (f4){0.f, 0.f, 0.f, 0.f};
    }

    // ---- staging roles (the tile's dequant work, split over all 8 waves)
    // K (waves 0-3): token 16*(wave & 1) + col of the tile, channel group grp,
    //   code pairs 8*kph .. 8*kph+7 (kph = wave >> 1); meta prep: channel
    //   pair pi2 of group g2 (as in the decode kernel), per wave.
    // V (waves 4-7): half vh = wave & 1, chunk col (8 channels), tokens
    //   16vh + 4grp + 2vp + {0, 1} (vp = (wave >> 1) & 1: which pair of the
    //   lane's MFMA token quad).
    const bool kwave = wave < 4;
    const int ktok = 16 * (wave & 1) + col;
    const int kph = (wave >> 1) & 1;
    const int g2 = lane >> 4, pi2 = lane & 15;
    const int kch_lo = 32 * g2 + kpair_chan<BK>(pi2, 0), kch_hi = 32 * g2 + kpair_chan<BK>(pi2, 1);
    const _Float16 nmul = (_Float16)(-magic_val(koff<BK>(pi2)));
    const int vh = wave & 1, vp = (wave >> 1) & 1;
    const int gv = (8 * col) / GV;
    unsigned char *kmeta = smem + 2 * kBuf + (wave & 3) * kPKmeta;
    const int tpb = p.T / kPTok;  // tiles per K block

    const __amdgpu_buffer_rsrc_t rkc = make_rsrc((const unsigned char *)p.kc + bh * p.n_warm * KR, (uint32_t)(p.n_warm * KR));
    const __amdgpu_buffer_rsrc_t rvc = make_rsrc((const unsigned char *)p.vc + bh * p.n_warm * VR, (uint32_t)(p.n_warm * VR));
    const __amdgpu_buffer_rsrc_t rks = make_rsrc(p.ks + bh * p.nblk * kPD, (uint32_t)(p.nblk * kPD * 2));
    const __amdgpu_buffer_rsrc_t rkz = make_rsrc(p.kz + bh * p.nblk * kPD, (uint32_t)(p.nblk * kPD * 2));
    const __amdgpu_buffer_rsrc_t rvs = make_rsrc(p.vs + bh * p.n_warm * NG, (uint32_t)(p.n_warm * NG * 2));
    const __amdgpu_buffer_rsrc_t rvz = make_rsrc(p.vz + bh * p.n_warm * NG, (uint32_t)(p.n_warm * NG * 2));
    const __amdgpu_buffer_rsrc_t rkh = make_rsrc(p.khot + bh * p.n_hot * kPD, (uint32_t)(p.n_hot * kPD * 2));
    const __amdgpu_buffer_rsrc_t rvh = make_rsrc(p.vhot + bh * p.n_hot * kPD, (uint32_t)(p.n_hot * kPD * 2));

    Masks<BK> km;
    km.init();
    Masks<BV> vmk;
    if (BV == BK) vmk = *(const Masks<BV> *)&km;
    else vmk.init();

    // Registers of the next tile, one set for every role:
    //   hot K: R[0..3] = 64 B of the token;  hot V: R[i] = 16 B of token i (i < 2);
    //   warm K: R[0] = code bytes, R[1] = s_lo, s_hi, z_lo, z_hi of the prep pair;
    //   warm V: R[0] = codes of tokens 0, 1 and their scales, R[1][0..1] = their zeros.
    u4 hraw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) hraw[i] = (u4){0u, 0u, 0u, 0u};

    // Global loads of tile t into the lane's registers (ranges past the end read 0).
    auto load_tile = [&](int t) {
        if (t < n_ht) {
            const uint32_t tok0 = (uint32_t)t * kPTok;
            if (kwave) {
                const uint32_t off = ((tok0 + ktok) * kPD + 32 * grp) * 2u;
#pragma unroll
                for (int i = 0; i < 4; ++i) hraw[i] = bld128(rkh, off + 16u * i);
            } else {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t off = ((tok0 + 16 * vh + 4 * grp + 2 * vp + i) * kPD + 8 * col) * 2u;
                    hraw[i] = bld128(rvh, off);
                }
            }
        } else {
            const int u = t - n_ht;
            const uint32_t tok0 = (uint32_t)u * kPTok;
            if (kwave) {
                const uint32_t off = (tok0 + ktok) * KR + grp * 4 * BK;
                if (BK == 4) hraw[0] = bld128(rkc, off);
                else if (BK == 3) {
                    const u3 x = bld96(rkc, off);
                    hraw[0] = (u4){x[0], x[1], x[2], 0u};
                } else {
                    const u2 x = bld64(rkc, off);
                    hraw[0] = (u4){x[0], x[1], 0u, 0u};
                }
                const uint32_t mrow = (uint32_t)(tpb == 1 ? u : u / tpb) * kPD;
                hraw[1] = (u4){bld16(rks, (mrow + kch_lo) * 2u), bld16(rks, (mrow + kch_hi) * 2u),
                               bld16(rkz, (mrow + kch_lo) * 2u), bld16(rkz, (mrow + kch_hi) * 2u)};
            } else {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t tk = tok0 + 16 * vh + 4 * grp + 2 * vp + i;
                    if (BV == 3) {
                        const uint32_t off = tk * VR + 3 * col;
                        const uint32_t d0 = bld32(rvc, off & ~3u);
                        const uint32_t d1 = (off & 3u) >= 2u ? bld32(rvc, (off & ~3u) + 4u) : 0u;
                        hraw[0][i] = __builtin_amdgcn_alignbyte(d1, d0, off & 3u);
                    } else if (BV == 4) {
                        hraw[0][i] = bld32(rvc, tk * VR + 4 * col);
                    } else {
                        hraw[0][i] = bld16(rvc, tk * VR + 2 * col);
                    }
                    hraw[0][2 + i] = bld16(rvs, (tk * NG + gv) * 2u);
                    hraw[1][i] = bld16(rvz, (tk * NG + gv) * 2u);
                }
            }
        }
    };

    // Dequantize the registers of tile t into LDS buffer `buf`.
    auto stage_tile = [&](int t, unsigned char *buf) {
        unsigned char *kt = buf, *vt = buf + kKTile, *vzt = buf + kKTile + kVTile;
        if (t < n_ht) {
            if (kwave) {
                uint32_t nat[16], pairs[16];
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t xe = hraw[q4][e];
                        nat[4 * q4 + e] = xe;
                    }
                hot_k_pairs<BK>(nat, pairs);
                u4 *dst = (u4 *)(kt + ktok * kKRow + grp * 64 + kph * 32);
                if (kph == 0) {
                    dst[0] = (u4){pairs[0], pairs[1], pairs[2], pairs[3]};
                    dst[1] = (u4){pairs[4], pairs[5], pairs[6], pairs[7]};
                } else {
                    dst[0] = (u4){pairs[8], pairs[9], pairs[10], pairs[11]};
                    dst[1] = (u4){pairs[12], pairs[13], pairs[14], pairs[15]};
                }
            } else {
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const uint32_t sel = (kk & 1) ? 0x07060302u : 0x05040100u;
                    *(uint32_t *)(vt + (((kk * 2 + vh) * 2 + vp) * 64 + lane) * 4) =
                        perm(hraw[1][kk / 2], hraw[0][kk / 2], sel);
                }
                // zeros operand of a hot tile: no zero-points; chunk row 15 takes ones (row sums)
                *(uint32_t *)(vzt + ((vh * 2 + vp) * 64 + lane) * 4) = col == 15 ? kOnes2 : 0u;
            }
            return;
        }
        if (kwave) {
            // K meta of the block: (s, -2^(10-o) s, z) per channel pair, shared through LDS
            const h2 s2v = as_h2(hraw[1][0] | (hraw[1][1] << 16));
            const h2 z2v = as_h2(hraw[1][2] | (hraw[1][3] << 16));
            const h2 n2 = s2v * (h2){nmul, nmul};
            const bool kfast = !__builtin_amdgcn_ballot_w64(!finite2(as_u32(n2)));
            uint32_t *kmw = (uint32_t *)kmeta;
            kmw[(0 * 4 + g2) * 16 + pi2] = as_u32(s2v);
            kmw[(1 * 4 + g2) * 16 + pi2] = as_u32(n2);
            kmw[(2 * 4 + g2) * 16 + pi2] = as_u32(z2v);
            __builtin_amdgcn_wave_barrier();
            KWin<BK> W;
            const uint32_t kraw[4] = {hraw[0][0], hraw[0][1], hraw[0][2], hraw[0][3]};
            k_windows<BK>(kraw, W);
            const u4 *srcm = (const u4 *)kmeta;
            uint32_t out[8];
            // pairs 8*kph + 4*c + e of this lane's group
            auto deq = [&](int ph) {
                if (kfast) {
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const int q4 = 2 * ph + c;
                        const u4 av = srcm[(0 * 4 + grp) * 4 + q4];
                        const u4 nv = srcm[(1 * 4 + grp) * 4 + q4];
                        const u4 zv = srcm[(2 * 4 + grp) * 4 + q4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int pi = 4 * q4 + e;
                            const uint32_t ae = av[e], ne = nv[e], ze = zv[e];
                            const uint32_t uu = (k_window_of<BK>(W, pi) & km.m[koff<BK>(pi)]) | magic2(koff<BK>(pi));
                            out[4 * c + e] = as_u32(pk_fma(as_h2(uu), as_h2(ae), as_h2(ne)) + as_h2(ze));
                        }
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const int q4 = 2 * ph + c;
                        const u4 av = srcm[(0 * 4 + grp) * 4 + q4];
                        const u4 zv = srcm[(2 * 4 + grp) * 4 + q4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int pi = 4 * q4 + e;
                            const uint32_t ae = av[e], ze = zv[e];
                            const uint32_t uu = (k_window_of<BK>(W, pi) & km.m[koff<BK>(pi)]) | magic2(koff<BK>(pi));
                            const _Float16 mv = (_Float16)magic_val(koff<BK>(pi));
                            out[4 * c + e] = as_u32((as_h2(uu) - (h2){mv, mv}) * as_h2(ae) + as_h2(ze));
                        }
                    }
                }
            };
            if (kph == 0) deq(0);
            else deq(1);
            u4 *dst = (u4 *)(kt + ktok * kKRow + grp * 64 + kph * 32);
            dst[0] = (u4){out[0], out[1], out[2], out[3]};
            dst[1] = (u4){out[4], out[5], out[6], out[7]};
            __builtin_amdgcn_wave_barrier();  // kmeta reads done before the next tile's writes
        } else {
            const h2 vs = as_h2(hraw[0][2] | (hraw[0][3] << 16));
            const h2 vz = as_h2(hraw[1][0] | (hraw[1][1] << 16));
            const _Float16 n0 = (_Float16)(-1024.0f);
            const bool vfast = !__builtin_amdgcn_ballot_w64(!finite2(as_u32(vs * (h2){n0, n0})));
            uint32_t win[VSlot<BV>::NW];
            v_windows<BV>(hraw[0][0], hraw[0][1], win);
            uint32_t vpair[8];
            if (vfast) {
                h2 vn[v_noffs<BV>()];
#pragma unroll
                for (int oi = 0; oi < v_noffs<BV>(); ++oi) {
                    const _Float16 m = (_Float16)(-magic_val(oi * v_ostep<BV>()));
                    vn[oi] = vs * (h2){m, m};
                }
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const uint32_t uu = (win[vwin<BV>(kk)] & vmk.m[voff<BV>(kk)]) | magic2(voff<BV>(kk));
                    vpair[kk] = as_u32(pk_fma(as_h2(uu), vs, vn[voff<BV>(kk) / v_ostep<BV>()]));
                }
            } else {
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const uint32_t uu = (win[vwin<BV>(kk)] & vmk.m[voff<BV>(kk)]) | magic2(voff<BV>(kk));
                    const _Float16 mv = (_Float16)magic_val(voff<BV>(kk));
                    vpair[kk] = as_u32((as_h2(uu) - (h2){mv, mv}) * vs);
                }
            }
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) *(uint32_t *)(vt + (((kk * 2 + vh) * 2 + vp) * 64 + lane) * 4) = vpair[kk];
            // chunk row 15 takes ones: that row of the zeros MFMA gives the row sums of P
            *(uint32_t *)(vzt + ((vh * 2 + vp) * 64 + lane) * 4) = col == 15 ? kOnes2 : as_u32(vz);
        }
    };

    // ---- the tile loop over the cache: load t+1 | MFMA on t | dequant t+1 | barrier
    const int tc_end = t_end < c_first ? t_end : c_first;
    if (t_begin < tc_end) {
        load_tile(t_begin);
        stage_tile(t_begin, smem);
    }
    __syncthreads();
    for (int t = t_begin; t < tc_end; ++t) {
        const int cur = (int)((t - t_begin) & 1);
        unsigned char *buf = smem + cur * kBuf;
        const bool more = t + 1 < tc_end;
        if (more) load_tile(t + 1);

        const bool hot = t < n_ht;
        const int tok0 = (hot ? t : t - n_ht) * kPTok;
        const int ntok = hot ? n_hot32 : n_warm32;
        const unsigned char *kt = buf, *vt = buf + kKTile, *vzt = buf + kKTile + kVTile;
        f4 sc[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            sc[0][h] = (f4){0.f, 0.f, 0.f, 0.f};
            sc[1][h] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const h8 a = *(const h8 *)(kt + (16 * h + col) * kKRow + grp * 64 + 16 * st);
                sc[0][h] = mfma_k32(a, qop[0][st], sc[0][h]);
                sc[1][h] = mfma_k32(a, qop[1][st], sc[1][h]);
            }
        }
        if (tok0 + kPTok > ntok) {  // ragged last tile: tokens past the tier score -inf
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (tok0 + 16 * h + 4 * grp + i >= ntok) {
                        sc[0][h][i] = -INFINITY;
                        sc[1][h][i] = -INFINITY;
                    }
        }
        h8 pop[2];
        pop[0] = softmax32(sm[0], sc[0][0], sc[0][1], sl2);
        pop[1] = softmax32(sm[1], sc[1][0], sc[1][1], sl2);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            const uint32_t *va = (const uint32_t *)(vt + (kk * 4 * 64 + lane) * 4);
            const h8 a = __builtin_bit_cast(h8, (u4){va[0], va[64], va[128], va[192]});
            sm[0].acc[kk] = mfma_k32(a, pop[0], sm[0].acc[kk]);
            sm[1].acc[kk] = mfma_k32(a, pop[1], sm[1].acc[kk]);
        }
        {
            // zeros MFMA: chunk rows 0-14 take the tile's zero-points (zero for hot tiles);
            // chunk row 15 takes ones, so its output is the row sum of P (l); the staging
            // wrote both.  Chunks 12-15 share one V group, so chunk 15's zero term is chunk 12's.
            const uint32_t *za = (const uint32_t *)(vzt + lane * 4);
            const h8 az = __builtin_bit_cast(h8, (u4){za[0], za[64], za[128], za[192]});
            sm[0].accz = mfma_k32(az, pop[0], sm[0].accz);
            sm[1].accz = mfma_k32(az, pop[1], sm[1].accz);
        }

        if (more) stage_tile(t + 1, smem + (cur ^ 1) * kBuf);
        __syncthreads();
    }

    // ---- the chunk's own tiles (when given and in this split): token rows in q's dtype,
    //      read like the hot tier's (bf16 converted to fp16, exact in fp16's range, as the
    //      queries are), a causal mask, no zero-points.  A loop of its own, so that its
    //      descriptors and row positions are live only here.
    const int tq_begin = t_begin > c_first ? t_begin : c_first;
    if (OWN && tq_begin < t_end) {
        const __amdgpu_buffer_rsrc_t rkq =
            make_rsrc((const uint16_t *)p.kcur + bh * p.n_cur * kPD, (uint32_t)(p.n_cur * kPD * 2));
        const __amdgpu_buffer_rsrc_t rvq =
            make_rsrc((const uint16_t *)p.vcur + bh * p.n_cur * kPD, (uint32_t)(p.n_cur * kPD * 2));
        int mrow[2];  // chunk position of each column group's row
#pragma unroll
        for (int rg = 0; rg < 2; ++rg) {
            const int r = r0 + 32 * wave + 16 * rg + col;
            mrow[rg] = (r < p.R ? r : r0) % p.M;
        }
        auto load_own = [&](int t) {
            const uint32_t tok0 = (uint32_t)(t - c_first) * kPTok;
            if (kwave) {
                const uint32_t off = ((tok0 + ktok) * kPD + 32 * grp) * 2u;
#pragma unroll
                for (int i = 0; i < 4; ++i) hraw[i] = bld128(rkq, off + 16u * i);
            } else {
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    hraw[i] = bld128(rvq, ((tok0 + 16 * vh + 4 * grp + 2 * vp + i) * kPD + 8 * col) * 2u);
            }
        };
        auto stage_own = [&](unsigned char *buf) {
            unsigned char *kt = buf, *vt = buf + kKTile;
            if (kwave) {
                uint32_t nat[16], pairs[16];
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
                    for (int e = 0; e < 4; ++e) nat[4 * q4 + e] = p.q_bf16 ? bf16x2_to_h2(hraw[q4][e]) : hraw[q4][e];
                hot_k_pairs<BK>(nat, pairs);
                u4 *dst = (u4 *)(kt + ktok * kKRow + grp * 64 + kph * 32);
                if (kph == 0) {
                    dst[0] = (u4){pairs[0], pairs[1], pairs[2], pairs[3]};
                    dst[1] = (u4){pairs[4], pairs[5], pairs[6], pairs[7]};
                } else {
                    dst[0] = (u4){pairs[8], pairs[9], pairs[10], pairs[11]};
                    dst[1] = (u4){pairs[12], pairs[13], pairs[14], pairs[15]};
                }
            } else {
                u4 w2[2];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) w2[i][e] = p.q_bf16 ? bf16x2_to_h2(hraw[i][e]) : hraw[i][e];
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const uint32_t sel = (kk & 1) ? 0x07060302u : 0x05040100u;
                    *(uint32_t *)(vt + (((kk * 2 + vh) * 2 + vp) * 64 + lane) * 4) = perm(w2[1][kk / 2], w2[0][kk / 2], sel);
                }
            }
        };
        load_own(tq_begin);
        stage_own(smem);
        __syncthreads();
        for (int t = tq_begin; t < t_end; ++t) {
            const int cur = (int)((t - tq_begin) & 1);
            const unsigned char *buf = smem + cur * kBuf;
            const bool more = t + 1 < t_end;
            if (more) load_own(t + 1);
            const int tok0 = (t - c_first) * kPTok;
            const unsigned char *kt = buf, *vt = buf + kKTile;
            f4 sc[2][2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                sc[0][h] = (f4){0.f, 0.f, 0.f, 0.f};
                sc[1][h] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    const h8 a = *(const h8 *)(kt + (16 * h + col) * kKRow + grp * 64 + 16 * st);
                    sc[0][h] = mfma_k32(a, qop[0][st], sc[0][h]);
                    sc[1][h] = mfma_k32(a, qop[1][st], sc[1][h]);
                }
            }
            // causal: position m sees chunk tokens 0..m (so none past the chunk's end)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int j = tok0 + 16 * h + 4 * grp + i;
                    if (j > mrow[0]) sc[0][h][i] = -INFINITY;
                    if (j > mrow[1]) sc[1][h][i] = -INFINITY;
                }
            h8 pop[2];
            pop[0] = softmax32(sm[0], sc[0][0], sc[0][1], sl2);
            pop[1] = softmax32(sm[1], sc[1][0], sc[1][1], sl2);
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const uint32_t *va = (const uint32_t *)(vt + (kk * 4 * 64 + lane) * 4);
                const h8 a = __builtin_bit_cast(h8, (u4){va[0], va[64], va[128], va[192]});
                sm[0].acc[kk] = mfma_k32(a, pop[0], sm[0].acc[kk]);
                sm[1].acc[kk] = mfma_k32(a, pop[1], sm[1].acc[kk]);
            }
            {
                // the row sums of P (chunk row 15 takes ones; no zero-points here)
                const u4 zw = col == 15 ? (u4){0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u}
                                        : (u4){0u, 0u, 0u, 0u};
                const h8 az = __builtin_bit_cast(h8, zw);
                sm[0].accz = mfma_k32(az, pop[0], sm[0].accz);
                sm[1].accz = mfma_k32(az, pop[1], sm[1].accz);
            }
            if (more) stage_own(smem + (cur ^ 1) * kBuf);
            __syncthreads();
        }
    }

    // ---- output (one split) or partials (decode split layout)
#pragma unroll
    for (int rg = 0; rg < 2; ++rg) {
        // l from chunk row 15 of the zeros MFMA (lanes of column group 3, element 3);
        // that chunk's zero term is chunk 12's (element 0 of the same lanes)
        const float l = wsum16(grp == 3 ? sm[rg].accz[3] : 0.f);
        if (grp == 3) sm[rg].accz[3] = sm[rg].accz[0];
        const int r = r0 + 32 * wave + 16 * rg + col;
        if (r >= p.R) continue;
        if (p.nsplit == 1) {
            const int hq = kvh * p.g + r / p.M, mq = r % p.M;
            const int64_t orow = ((int64_t)(b * p.Hq + hq) * p.M + mq) * kPD;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float o[8];
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) o[kk] = (sm[rg].acc[kk][i] + sm[rg].accz[i]) / l;
                uint32_t w[4];
                if (p.q_bf16) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        w[e] = (uint32_t)f32_to_bf16_rne(o[2 * e]) | ((uint32_t)f32_to_bf16_rne(o[2 * e + 1]) << 16);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = as_u32((h2){(_Float16)o[2 * e], (_Float16)o[2 * e + 1]});
                }
                *(u4 *)((uint16_t *)p.out + orow + 8 * (4 * grp + i)) = (u4){w[0], w[1], w[2], w[3]};
            }
        } else {
            const int chunk = r / 16, rr = r % 16;
            float *part = p.part + ((bh * p.nchunk + chunk) * p.nsplit + split) * (int64_t)(p.prows * (kPD + 4)) +
                          rr * (kPD + 4);
            if (grp == 0) {
                part[0] = sm[rg].m2;
                part[1] = l;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f4 *dst = (f4 *)(part + 4 + 8 * (4 * grp + i));
                dst[0] = (f4){sm[rg].acc[0][i] + sm[rg].accz[i], sm[rg].acc[1][i] + sm[rg].accz[i],
                              sm[rg].acc[2][i] + sm[rg].accz[i], sm[rg].acc[3][i] + sm[rg].accz[i]};
                dst[1] = (f4){sm[rg].acc[4][i] + sm[rg].accz[i], sm[rg].acc[5][i] + sm[rg].accz[i],
                              sm[rg].acc[6][i] + sm[rg].accz[i], sm[rg].acc[7][i] + sm[rg].accz[i]};
            }
        }
    }
}

int prefill_lds_bytes() { return kPLds; }

template <int BK, int BV, int NG>
static hipError_t launch_prefill(const PrefillParams &p, hipStream_t s) {
    const unsigned nwg = (unsigned)(p.B * p.Hkv * p.nsplit * p.n_row_tiles);
    if (p.kcur && p.n_cur > 0)
        hipLaunchKernelGGL((prefill_kernel<BK, BV, NG, true>), dim3(nwg), dim3(kPThreads), kPLds, s, p);
    else
        hipLaunchKernelGGL((prefill_kernel<BK, BV, NG, false>), dim3(nwg), dim3(kPThreads), kPLds, s, p);
    return hipGetLastError();
}

template <int BK, int BV>
static hipError_t launch_prefill_ng(const PrefillParams &p, hipStream_t s) {
    if (p.Gv == 32) return launch_prefill<BK, BV, 4>(p, s);
    if (p.Gv == 64) return launch_prefill<BK, BV, 2>(p, s);
    if (p.Gv == 128) return launch_prefill<BK, BV, 1>(p, s);
    return hipErrorInvalidValue;
}

hipError_t prefill_launch(const PrefillParams &p, hipStream_t s) {
    hipError_t e = hipErrorInvalidValue;
#define AKV_PKV(a, c) \
    if (p.bits_k == a && p.bits_v == c) e = launch_prefill_ng<a, c>(p, s);
    AKV_PKV(2, 2) AKV_PKV(2, 3) AKV_PKV(2, 4) AKV_PKV(3, 2) AKV_PKV(3, 3) AKV_PKV(3, 4) AKV_PKV(4, 2) AKV_PKV(4, 3)
    AKV_PKV(4, 4)
#undef AKV_PKV
    if (e != hipSuccess || p.nsplit == 1) return e;
    DecodeParams d{};
    d.B = p.B; d.Hq = p.Hq; d.Hkv = p.Hkv; d.M = p.M; d.D = kPD; d.g = p.g; d.R = p.R;
    d.nchunk = p.nchunk; d.prows = p.prows; d.nsplit = p.nsplit;
    d.part = p.part;
    d.out = (_Float16 *)p.out;
    d.out_bf16 = p.q_bf16;
    return decode_reduce_launch(d, s);
}

}  // namespace akv
