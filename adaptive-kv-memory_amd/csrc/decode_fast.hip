// Split-K fused dequant-attention over the block-affine warm tier, streamed
// through LDS: the decode kernel of the 32k-context workload.
//
// Scope: head_dim 128, K blocks of T tokens with T a multiple of 32, V groups
// of G = 32, 64 or 128 channels, 2/3/4 bits for K and V, and (variant OUT, V
// groups of 32) up to 4 fp16 outlier channels per block.  Variant LEG reads the
// legacy per-token-group layout (the reference's public legacy ops and
// PackedKVArena): 2 or 4 bits, one group size of 32 / 64 / 128 channels for K
// and V, fp16 scales and zeros per (token, group), a warm tier per head or one
// shared by all, rows w_stride apart; its K meta is loaded like V's, each lane's
// 32 K channels share one (s, z), and K and V values are round16((c - offset) s
// + z) in one fma (offset = half_max in the symmetric branch, else 0).  Other
// shapes use decode_split_kernel (decode.hip).
//
// Work split: a 1-D grid over (split, kv-head, batch * row-chunk), renumbered
// so that each XCD gets a contiguous run of items; a workgroup of 12 waves (8
// for OUT > 1) owns one (batch, kv-head, row chunk of 16 query rows) and one token
// range: warm 32-token units first, then hot 16-token tiles (each two items:
// its K and its V half).  A wave takes its first item by its index and the
// next ones from a workgroup counter in LDS, through a private ring of NS LDS
// slots filled by buffer loads that write LDS directly (16 B per lane).  A
// unit's arrays (K codes, V codes, K scale, K zero, V scale, V zero, and the
// outlier values and indices) are each one contiguous byte range, so a slot
// fills with a few wave-wide loads whose offsets are scalars; ranges past the
// end of a (batch, kv-head) read as zero (buffer range check), which keeps
// ragged tails in bounds.  The loads of the younger slots stay in flight while
// the oldest is computed.
//
// Per 32-token warm unit a wave does:
//   QK:  S^T[16 tok x 16 rows] = K . Q^T for both 16-token halves, 4 x
//        v_mfma_f32_16x16x32_f16 each.  Lane (token l%16, channel group l/16)
//        builds its 32 K values from byte-permuted windows of its packed row:
//        one and-or puts a code pair into the mantissas of two fp16 numbers
//        2^(10-o) + c (o = the code's bit offset in the window), one packed
//        fma with (s, -2^(10-o) s) gives round16(c*s) exactly, one packed add
//        gives round16(. + z): the reference's fp16 dequant bit for bit.  The
//        per-channel (s, n, z) pairs of the block are prepared per unit in
//        LDS; the query operand is staged once per workgroup in LDS.
//   softmax: online over the 32 tokens, log2 domain, lazy rescale (threshold
//        2^8); probabilities enter PV as fp16 scaled by 2^7.
//   PV:  O^T[16 chunks x 16 rows] += V^T . P^T over the 32 tokens, 8 x
//        v_mfma_f32_16x16x32_f16.  Lane (chunk l%16 of 8 channels, tokens
//        4(l/16)..+3 of each half) pairs two tokens per dword with byte
//        permutes and shifts; one and-or and one packed fma give round16(c*s)
//        with the token's scale of its group.  The zero-points enter through
//        one more MFMA per unit that accumulates sum_t P * z(token, group),
//        added to every channel of the group at the end (so V skips the second
//        fp16 rounding of the reference's dequant: the output stays within the
//        attention tolerance).
//   OUT: the stored fp16 value of an outlier channel replaces its dequantized
//        value.  K: q[c] (value - dequant) joins the scores (q[c] value alone
//        when the channel's block meta is zero, as the quantizer leaves it).
//        V, one outlier channel per block: the value goes into the PV operand in
//        place of the channel's dequantized codes, and one MFMA takes the zero
//        term the zero-point MFMA added back out; more channels: three exact
//        MFMAs per channel add sum_t P (value - round16(code s) - z).
// The waves merge in LDS; each workgroup writes its (m, l, acc) partial and
// counts its arrival; the last workgroup of a (batch, kv-head, row chunk)
// merges the partials and writes the output and the row statistics.
//
// A block whose scales would overflow -2^(10-o) s in fp16 (|s| >= 64) takes
// a slower exact path: the code is recovered as an fp16 integer, then
// round16(c * s) and round16(. + z) are two packed ops.
#include <atomic>

#include "akv_common.h"
#include "decode.h"
#include "tile_common.h"

namespace akv {

// ---- per-wave timeline, recorded only by the timeline build of the library
// (make timeline: -DAKV_TIMELINE).  Words per wave (blockIdx.x * waves + wave):
// 0 start, 1 first item's data in LDS, 2 warm items done, 3 all items done,
// 4 partial written and acknowledged, 5 arrival counted (ticks x 4 + role:
// 0 not last, 1 last, 2 last with every partial from its XCD), 6 merge done (wave 0
// of the merging workgroup), 7 items taken, 8 ticks waiting for ring data, 9 XCC id,
// 10 first load issued, 11 waves merged in LDS, 12 merger's partial loads done (thread 0),
// 13 start barrier passed.  Times are s_memrealtime ticks
// (100 MHz).  The words are kept in registers and written once, by lane 0, where the
// wave leaves the kernel (AKV_TL_FLUSH), so no timeline store waits among the kernel's
// own memory operations; the values carry threadIdx.x & 1 (0 on lane 0) so that they
// live in vector registers and leave through vector stores.
#ifdef AKV_TIMELINE
constexpr int kTlWords = 16, kTlCap = 1 << 17;
__device__ unsigned long long g_akv_timeline[kTlCap];
#define AKV_TL(k, v) (tl_v[(k)] = (unsigned long long)(v) + (threadIdx.x & 1u))
#define AKV_TL_NOW() __builtin_amdgcn_s_memrealtime()
#define AKV_TL_FLUSH()                                                        \
    do {                                                                      \
        if (lane == 0 && tl_base + kTlWords <= kTlCap)                        \
            for (int tl_k = 0; tl_k < kTlWords; ++tl_k) g_akv_timeline[tl_base + tl_k] = tl_v[tl_k]; \
    } while (0)
#else
#define AKV_TL(k, v) ((void)0)
#define AKV_TL_NOW() 0ull
#define AKV_TL_FLUSH() ((void)0)
#endif

namespace {

constexpr int kD = 128;
#ifndef AKV_FAST_WAVES
#define AKV_FAST_WAVES 12
#endif
#ifndef AKV_FAST_NS
#define AKV_FAST_NS 2
#endif
constexpr int kWaves = AKV_FAST_WAVES;  // waves per workgroup (one workgroup per CU, 3 per SIMD)
constexpr int kUnit = 32;               // warm tokens per ring slot
constexpr int kNS = AKV_FAST_NS;        // ring slots per wave (deeper rings only lengthen the tail)
// OUT selects the outlier-channel variant: 0 none; 1 exactly one channel per
// block (the one-channel paths only: 147-156 VGPRs, so 12 waves with 2 slots
// like OUT = 0); kMaxOut up to 4 channels, whose general corrections hold more
// state per lane: 8 waves (2 per SIMD, twice the registers each) with 3 slots.
#ifndef AKV_FAST_WAVES_OUT
#define AKV_FAST_WAVES_OUT 8
#endif
#ifndef AKV_FAST_NS_OUT
#define AKV_FAST_NS_OUT 3
#endif
constexpr int kWavesOut = AKV_FAST_WAVES_OUT, kNSOut = AKV_FAST_NS_OUT;
template <int OUT> struct FastCfg {
    static constexpr int NW = OUT > 1 ? kWavesOut : kWaves, NS = OUT > 1 ? kNSOut : kNS;
};
constexpr int kLdsCap = 160 * 1024;  // LDS of one CU
constexpr int kKmetaBytes = 3 * 4 * 16 * 4;  // [s | n | z][group][pair] u32
constexpr int kHotLoads = 4;         // 16 tokens x 256 B = 4 KiB = 4 wave loads
constexpr int kQldsBytes = 16 * kD * 2;  // the workgroup's 16 query rows (fp16)
constexpr int kAccRow = kD + 4;      // fp32 row of the end-of-split merge in LDS (the pad spreads a
                                     // wave's 64 row/chunk writes over the banks)
constexpr int kMaxOut = 4;            // outlier channels per block the fast kernel takes
constexpr int kOutBytes = 2 * (kUnit * kMaxOut * 2) + 2 * 32;  // K/V outlier values + K/V indices
template <int BK, int BV, int NG, int OUT, bool LEG>
struct WarmLayout {
    static constexpr int KR = 16 * BK, VR = 16 * BV;  // packed row bytes (D = 128)
    static constexpr int KCB = kUnit * KR, VCB = kUnit * VR;
    static constexpr int VMB = 64 * NG;               // V scale (or zero) bytes of 32 tokens
    // K scale (or zero) bytes of a unit: the block's row of D channels, or (LEG) the 32
    // tokens' rows of NG groups, laid out like V's
    static constexpr int KMB = LEG ? VMB : 256;
    static constexpr int NKC = (KCB + 1023) / 1024, NVC = (VCB + 1023) / 1024;
    // full-lane load patterns (dma_lean) where the range sizes allow them
    static constexpr bool LEAN_C = dma_lean_ok<KCB>() && dma_lean_ok<VCB>();
    static constexpr bool LEAN_VM = dma_lean_ok<64 * NG>();
    static constexpr int NLOAD = (LEAN_C ? dma_count<KCB>() + dma_count<VCB>() : NKC + NVC) +
                                 (LEG ? (LEAN_VM ? 2 * dma_count<64 * NG>() : 2) : 2) +
                                 (LEAN_VM ? 2 * dma_count<64 * NG>() : 2) + (OUT ? 4 : 0);
    static constexpr int KC = 0, VC = KCB, KS = KCB + VCB, KZ = KS + KMB, VS = KZ + KMB, VZ = VS + VMB;
    // outlier channels: fp16 values [token][n_out] of K and V, int64 channel indices of the block
    static constexpr int KO = VZ + VMB, VO = KO + kUnit * kMaxOut * 2, KI = VO + kUnit * kMaxOut * 2, VI = KI + 32;
    static constexpr int BYTES = OUT ? VI + 32 : VZ + VMB;
};

struct WarmRes {
    u4 kc, vc, ks, kz, vs, vz;
    u4 ko, vo, ki, vi;  // outlier values and indices
};

template <int BK, int BV, int NG, int OUT, bool LEG>
__device__ __forceinline__ void issue_warm(const WarmRes &R, unsigned char *slot, int lane, int u, int T, int tshift,
                                           int n_out) {
    using L = WarmLayout<BK, BV, NG, OUT, LEG>;
    const uint32_t v16 = (uint32_t)lane * 16u, v4 = (uint32_t)lane * 4u;
    const uint32_t base = lds_addr(slot);
    if constexpr (L::LEAN_C) {
        dma_lean<L::KCB>(R.kc, base + L::KC, (uint32_t)u * L::KCB, v16, v4);
        dma_lean<L::VCB>(R.vc, base + L::VC, (uint32_t)u * L::VCB, v16, v4);
    } else {
#pragma unroll
        for (int i = 0; i < L::NKC; ++i)
            dma16(R.kc, base + L::KC + 1024 * i, v16, (uint32_t)u * L::KCB + 1024u * i, lane_mask(L::KCB - 1024 * i));
#pragma unroll
        for (int i = 0; i < L::NVC; ++i)
            dma16(R.vc, base + L::VC + 1024 * i, v16, (uint32_t)u * L::VCB + 1024u * i, lane_mask(L::VCB - 1024 * i));
    }
    // K block of the unit: T / 32 units per block (a shift when that is a power of two)
    const uint32_t blk = tshift >= 0 ? (uint32_t)u >> tshift : (uint32_t)((u * kUnit) / T);
    if constexpr (LEG) {  // per-token rows of K meta, as V's
        if constexpr (L::LEAN_VM) {
            dma_lean<64 * NG>(R.ks, base + L::KS, (uint32_t)u * (uint32_t)L::VMB, v16, v4);
            dma_lean<64 * NG>(R.kz, base + L::KZ, (uint32_t)u * (uint32_t)L::VMB, v16, v4);
        } else {
            dma16(R.ks, base + L::KS, v16, (uint32_t)u * (uint32_t)L::VMB, lane_mask(L::VMB));
            dma16(R.kz, base + L::KZ, v16, (uint32_t)u * (uint32_t)L::VMB, lane_mask(L::VMB));
        }
    } else {
        const uint32_t kmrow = blk * 256u;
        dma_lean<256>(R.ks, base + L::KS, kmrow, v16, v4);
        dma_lean<256>(R.kz, base + L::KZ, kmrow, v16, v4);
    }
    if constexpr (L::LEAN_VM) {
        dma_lean<64 * NG>(R.vs, base + L::VS, (uint32_t)u * (uint32_t)L::VMB, v16, v4);
        dma_lean<64 * NG>(R.vz, base + L::VZ, (uint32_t)u * (uint32_t)L::VMB, v16, v4);
    } else {
        dma16(R.vs, base + L::VS, v16, (uint32_t)u * (uint32_t)L::VMB, lane_mask(L::VMB));
        dma16(R.vz, base + L::VZ, v16, (uint32_t)u * (uint32_t)L::VMB, lane_mask(L::VMB));
    }
    if (OUT) {
        const uint32_t ob = (uint32_t)(kUnit * n_out * 2);  // 64 n_out bytes of values per unit
        const uint64_t im = lane_mask((n_out * 8 + 15) & ~15);
        dma16(R.ko, base + L::KO, v16, (uint32_t)u * ob, lane_mask((int)ob));
        dma16(R.vo, base + L::VO, v16, (uint32_t)u * ob, lane_mask((int)ob));
        dma16(R.ki, base + L::KI, v16, blk * (uint32_t)(n_out * 8), im);
        dma16(R.vi, base + L::VI, v16, blk * (uint32_t)(n_out * 8), im);
    }
}

__device__ __forceinline__ void issue_hot(u4 r, unsigned char *slot, int lane, int tile) {
    static_assert(dma_count<4096>() == kHotLoads, "hot tile loads");
    dma_lean<4096>(r, lds_addr(slot), (uint32_t)tile * 4096u, (uint32_t)lane * 16u, (uint32_t)lane * 4u);
}

// Raw logits q.k of 4 consecutive tokens of one row (the weights kernels take them to
// the log2 domain): one 16-byte store when all 4 are valid and the row offset is
// 16-byte aligned (vec), else one per token.  The 16-byte stores write through to the
// device coherence point (cache policy sc1): the stash leaves during the kernel instead
// of in the end-of-kernel L2 write-back (measured 0.35 us per layer faster at the 32k
// workload).  Whole warm units take a cheaper path in the loop itself.
__device__ __forceinline__ void stash4(const DecodeParams &p, int64_t strow, int row_valid, int64_t n0, f4 s,
                                       int nvalid, bool vec, __amdgpu_buffer_rsrc_t srs, int64_t sbase) {
    if (!p.stash || !row_valid) return;
    float *dst = p.stash + strow + n0;
    if (vec && nvalid >= 4) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, s), srs, (int)((strow + n0 - sbase) * 4), 0, 16);
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (i < nvalid) dst[i] = s[i];
}

// Online merge of the nsplit partials (m, l, acc) of row rr, channels 4 c4 .. +3,
// loaded with cache policy CP.
template <int CP>
__device__ __forceinline__ void merge_partials(__amdgpu_buffer_rsrc_t prs, int nsplit, int64_t pstride, int rr, int c4,
                                               float &M, float &L, f4 &a) {
    constexpr int PS = 128 + 4, KS = 16;  // partial row; splits per batch of loads
    for (int s0 = 0; s0 < nsplit; s0 += KS) {
        f2 ml[KS];
        f4 xs[KS];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const int off = (int)(((s0 + k) * pstride + rr * PS) * 4);
            const bool in = s0 + k < nsplit;
            ml[k] = in ? __builtin_bit_cast(f2, __builtin_amdgcn_raw_buffer_load_b64(prs, off, 0, CP)) : (f2){-INFINITY, 0.f};
            xs[k] = in ? __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(prs, off + 16 + 16 * c4, 0, CP))
                       : (f4){0.f, 0.f, 0.f, 0.f};
        }
        float nm = M;
#pragma unroll
        for (int k = 0; k < KS; ++k) nm = fmaxf(nm, ml[k][0]);
        if (nm == -INFINITY) continue;
        const float fo = (M == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(M - nm);
        a *= fo;
        L *= fo;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const float f = (ml[k][0] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(ml[k][0] - nm);
            a += f * xs[k];
            L += f * ml[k][1];
        }
        M = nm;
    }
}

}  // namespace


// Work item kinds of a ring slot.
constexpr int kNone = 0, kWarm = 1, kHotK = 2, kHotV = 3;

// Loads still in flight behind the oldest ring slot, given how many of the
// younger slots hold a warm unit (nw) or a hot half (nh); nw + nh <= MAXY.
template <int NLW, int NLH, int MAXY, int W = 0, int H = 0>
__device__ __forceinline__ void wait_younger(int nw, int nh) {
    if constexpr (W + H <= MAXY) {
        if (nw == W && nh == H) {
            wait_vm<W * NLW + H * NLH>();
            return;
        }
    }
    if constexpr (H < MAXY) wait_younger<NLW, NLH, MAXY, W, H + 1>(nw, nh);
    else if constexpr (W < MAXY) wait_younger<NLW, NLH, MAXY, W + 1, 0>(nw, nh);
    else wait_vm<0>();
}

template <int BK, int BV, int NG, int NS, int OUT, bool LEG>
__global__ __launch_bounds__(64 * FastCfg<OUT>::NW)
__attribute__((amdgpu_waves_per_eu(FastCfg<OUT>::NW / 4, FastCfg<OUT>::NW / 4)))
void decode_fast_kernel(const DecodeParams p) {
    constexpr int NW = FastCfg<OUT>::NW;  // waves of the workgroup
    static_assert(NS >= 2 && NS <= 4, "ring depth");
    static_assert(!(LEG && OUT), "the legacy layout has no outlier channels");
    using L = WarmLayout<BK, BV, NG, OUT, LEG>;
    constexpr int KSTEPS = kD / 32;
    constexpr int NLW = L::NLOAD;     // loads of a warm unit
    constexpr int NLH = kHotLoads;    // loads of a hot half
    constexpr int GV = kD / NG;       // V group size

    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, grp = lane >> 4;
    // Workgroup -> (split, kv-head, batch x row chunk).  Workgroups are handed to
    // the 8 XCDs round-robin by linear id; the order below gives each XCD a
    // contiguous run of (pair, split) items, so all splits of a pair usually share
    // one L2 and the in-kernel split merge reads their partials from it.
    int wid = (int)blockIdx.x;
    {
        const int nwg = (int)gridDim.x;
        if (nwg % 8 == 0) wid = (wid % 8) * (nwg / 8) + wid / 8;
    }
#ifdef AKV_TIMELINE
    const int tl_base = ((int)blockIdx.x * NW + wave) * kTlWords;
    unsigned long long tl_v[kTlWords];
#pragma unroll
    for (int tl_k = 0; tl_k < kTlWords; ++tl_k) tl_v[tl_k] = 0;
    AKV_TL(0, AKV_TL_NOW());
    unsigned long long tl_wait = 0;
    int tl_items = 0;
#endif
    // (split, kv-head, batch x row chunk) of the workgroup, by multiply-shift division
    const int q1 = (int)fast_div((uint32_t)wid, p.fd_nsplit);
    const int split = wid - q1 * p.nsplit;
    const int bz = (int)fast_div((uint32_t)q1, p.fd_hkv);
    const int kvh = q1 - bz * p.Hkv;
    const int b = (int)fast_div((uint32_t)bz, p.fd_nchunk), chunk = bz - b * p.nchunk;
    const int row0 = chunk * 16;
    const int nrows = min(16, p.R - row0);
    const int slot_bytes = p.slot_bytes;
    unsigned char *ring = smem + wave * (NS * slot_bytes + kKmetaBytes);
    unsigned char *kmeta = ring + NS * slot_bytes;
    unsigned *work = (unsigned *)(smem + NW * (NS * slot_bytes + kKmetaBytes));  // item counter
    // the 16 query rows in natural channel order (fp16): outlier-channel corrections
    _Float16 *qn_lds = (_Float16 *)(smem + NW * (NS * slot_bytes + kKmetaBytes) + 16);

    const int r = row0 + col;
    const int row_valid = col < nrows;
    const int rc = row_valid ? r : row0;
    const int rq = (int)fast_div((uint32_t)rc, p.fd_m);
    const int hq = kvh * p.g + rq, mq = rc - rq * p.M;
    const int64_t strow = ((int64_t)(b * p.Hq + hq) * p.M + mq) * p.N;
    const int64_t bh = (int64_t)b * p.Hkv + kvh;
    const float sl2 = p.scale_log2;
    // legacy layout: the symmetric branch ((code - half_max) s) per K / V, forced or detected
    // by an earlier kernel on this stream
    int symk = 0, symv = 0;
    if constexpr (LEG) {
        symk = __builtin_amdgcn_readfirstlane(p.sym_flags ? p.sym_flags[0] : p.legacy_sym);
        symv = __builtin_amdgcn_readfirstlane(p.sym_flags ? p.sym_flags[1] : p.legacy_sym);
    }
    // code offsets of the legacy symmetric branch (0 otherwise)
    const _Float16 hofk = (_Float16)(symk ? p.half_max_k : 0.f), hofv = (_Float16)(symv ? p.half_max_v : 0.f);
    const int64_t warm_base = p.hot_first ? p.n_hot : 0;  // logical position of warm token 0
    const int64_t hot_base = p.hot_first ? 0 : p.n_warm;
    // the stash rows are N floats apart: 16-byte stores need N and the segment base divisible by 4
    // the stash rows of this (batch, kv-head) as one buffer (byte offsets below 2^31)
    const int64_t sbase = ((int64_t)(b * p.Hq + kvh * p.g) * p.M) * p.N;
    const bool st_buf_ok = (int64_t)p.R * p.N * 4 < ((int64_t)1 << 31);
    const __amdgpu_buffer_rsrc_t srs =
        make_rsrc(p.stash ? p.stash + sbase : p.stash, st_buf_ok ? (uint32_t)(p.R * p.N * 4) : 0u);
    const bool st_vec_w = st_buf_ok && p.N % 4 == 0 && warm_base % 4 == 0,
               st_vec_h = st_buf_ok && p.N % 4 == 0 && hot_base % 4 == 0;
    // byte offset of the lane's 4 logits of warm token 0 within those rows (a whole unit's
    // stores add its token offset as the scalar operand)
    const uint32_t st_w_voff = st_vec_w ? (uint32_t)((strow - sbase + warm_base + 4 * grp) * 4) : 0u;

    // this workgroup's items: warm 32-token units, then hot 16-token tiles (the
    // cheap hot items come last and even out the waves' finishing times)
    const int nw = (int)p.n_warm, nh = (int)p.n_hot;
    const int w_begin = min(split * (int)p.wsplit_len, nw), w_end = min(w_begin + (int)p.wsplit_len, nw);
    const int h_begin = min(split * (int)p.hsplit_len, nh), h_end = min(h_begin + (int)p.hsplit_len, nh);
    const int u_first = w_begin / kUnit, n_wu = w_end > w_begin ? (w_end + kUnit - 1) / kUnit - u_first : 0;
    const int t_first = h_begin / 16, n_ht = h_end > h_begin ? (h_end + 15) / 16 - t_first : 0;
    const int n_items = n_wu + n_ht;
    // items 0 .. NW-1 go to waves 0 .. NW-1; the counter hands out the rest
    if (threadIdx.x == 0) *work = (unsigned)NW;

    WarmRes R;
    {
        const uint32_t nwu = (uint32_t)p.n_warm;
        // first token row of this (batch, kv-head)'s warm tier: dense per (batch, kv-head) for the
        // block-affine layout; for the legacy layout one tier shared by all, one per kv head
        // (shared by the batch) or one per (batch, kv head), w_stride rows apart
        const int64_t wrow =
            LEG ? (p.warm_heads == 1 ? 0 : p.warm_heads == p.Hkv ? (int64_t)kvh : bh) * p.w_stride : bh * p.n_warm;
        R.kc = rsrc4((const unsigned char *)p.kc + wrow * L::KR, nwu * L::KR);
        R.vc = rsrc4((const unsigned char *)p.vc + wrow * L::VR, nwu * L::VR);
        // Per-token meta: with 4 groups a unit's rows are loaded a dword per lane, and every
        // dword ends on a token; with 1 or 2 groups they come in 16-byte loads, and a load that
        // crosses the end of the range may be dropped whole by the range check, so the range is
        // rounded up to 16 bytes (the base is 16-byte aligned, so the last load lies in the
        // page of its first byte) and the rows past the tier are cleared in LDS before use.
        const uint32_t mrec = NG == 4 ? nwu * 8u : (nwu * NG * 2 + 15u) & ~15u;
        if (LEG) {
            R.ks = rsrc4((const _Float16 *)p.ks + wrow * NG, mrec);
            R.kz = rsrc4((const _Float16 *)p.kz + wrow * NG, mrec);
        } else {
            R.ks = rsrc4((const _Float16 *)p.ks + bh * p.nblk * kD, (uint32_t)(p.nblk * kD * 2));
            R.kz = rsrc4((const _Float16 *)p.kz + bh * p.nblk * kD, (uint32_t)(p.nblk * kD * 2));
        }
        R.vs = rsrc4((const _Float16 *)p.vs + wrow * NG, mrec);
        R.vz = rsrc4((const _Float16 *)p.vz + wrow * NG, mrec);
        if (OUT) {
            const int no = OUT == 1 ? 1 : p.n_out;
            R.ko = rsrc4(p.k_odata + bh * p.n_warm * no, nwu * (uint32_t)no * 2);
            R.vo = rsrc4(p.v_odata + bh * p.n_warm * no, nwu * (uint32_t)no * 2);
            R.ki = rsrc4(p.k_oidx + (int64_t)b * p.nblk * no, (uint32_t)(p.nblk * no * 8));
            R.vi = rsrc4(p.v_oidx + (int64_t)b * p.nblk * no, (uint32_t)(p.nblk * no * 8));
        }
    }
    const u4 rkh = rsrc4(p.khot + bh * p.h_stride * kD, (uint32_t)(p.n_hot * kD * 2));
    const u4 rvh = rsrc4(p.vhot + bh * p.h_stride * kD, (uint32_t)(p.n_hot * kD * 2));

    // ---- the ring: a queue of NS slots, oldest first; a hot item is two units (K, then V)
    int qk[NS], qi[NS];
    int pend = -1;         // hot tile whose V half is still to be issued
    bool claimed = false;  // the first item is the wave's own; later ones come from the counter
    auto next_unit = [&](int &k, int &id) {
        if (pend >= 0) {
            k = kHotV;
            id = pend;
            pend = -1;
            return;
        }
        unsigned it = (unsigned)wave;
        if (claimed) {
            if (lane == 0) it = atomicAdd(work, 1u);
            it = __builtin_amdgcn_readfirstlane(it);
        }
        claimed = true;
        if ((int)it >= n_items) {
            k = kNone;
            id = 0;
        } else if ((int)it < n_wu) {
            k = kWarm;
            id = u_first + (int)it;
        } else {
            k = kHotK;
            id = t_first + (int)it - n_wu;
            pend = id;
        }
    };
    auto issue = [&](int k, int id, unsigned char *slot) {
        if (k == kWarm) issue_warm<BK, BV, NG, OUT, LEG>(R, slot, lane, id, p.T, p.tshift, OUT == 1 ? 1 : p.n_out);
        else if (k == kHotK) issue_hot(rkh, slot, lane, id);
        else if (k == kHotV) issue_hot(rvh, slot, lane, id);
    };
    // Only the first slot is filled up front, with the 16 query rows of the workgroup
    // (4 KiB, rows past the chunk read as zeros) in the last slot beside it: every wave's
    // first unit is in the memory queue before any wave's second, so compute starts as
    // soon as a first unit lands; the other slots fill once it has.
    next_unit(qk[0], qi[0]);
    AKV_TL(10, AKV_TL_NOW());
    issue(qk[0], qi[0], ring);
    {
        // the chunk's rows r are query rows (kvh * g + r / M, r % M): consecutive in q
        const int64_t qrow0 = ((int64_t)(b * p.Hq + kvh * p.g) * p.M + row0) * kD;
        issue_hot(rsrc4(p.q + qrow0, (uint32_t)(nrows * kD * 2)), ring + (NS - 1) * slot_bytes, lane, 0);
    }
#pragma unroll
    for (int s2 = 1; s2 < NS; ++s2) qk[s2] = kNone;

    Soft stt;
    stt.m2 = -INFINITY;
    stt.l = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) stt.acc[j] = (f4){0.f, 0.f, 0.f, 0.f};
    stt.accz = (f4){0.f, 0.f, 0.f, 0.f};

    Masks<BK> km;
    km.init();
    Masks<BV> vmk;
    if (BV == BK) vmk = *(const Masks<BV> *)&km;
    else vmk.init();
    // K meta prep role of this lane: (group g2, pair pi2)
    const int g2 = lane >> 4, pi2 = lane & 15;
    const int kch_lo = 32 * g2 + kpair_chan<BK>(pi2, 0), kch_hi = 32 * g2 + kpair_chan<BK>(pi2, 1);
    const _Float16 nmul = (_Float16)(-magic_val(koff<BK>(pi2)));
    // V role: chunk col and its group; lane parts of the slot offsets
    const int gv = (8 * col) / GV;
    const int k_lane = L::KC + col * L::KR + grp * 4 * BK;
    const int v_lane = L::VC + 4 * grp * L::VR + (BV == 3 ? 3 * col : BV == 4 ? 4 * col : 2 * col);
    const int vm_lane = (4 * grp * NG + gv) * 2;

    __syncthreads();  // the item counter is in LDS before any wave claims from it
    AKV_TL(13, AKV_TL_NOW());
    wait_vm<0>();  // the first item and the query rows have landed
    AKV_TL(1, AKV_TL_NOW());
    // Q operand (B of QK): lane = (row col, channel group grp), in the channel order the
    // warm code pairs come out in (hot K is permuted to match); it stays in registers for
    // the whole range (16 VGPRs).  The outlier variants also keep the rows in natural
    // channel order in LDS (every wave writes the same values there).
    h8 qreg[KSTEPS];
    {
        const unsigned char *qs = ring + (NS - 1) * slot_bytes;
        uint32_t nat[16], pairs[16];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const u4 x = *(const u4 *)(qs + col * 256 + grp * 64 + 16 * q4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t xe = x[e];
                nat[4 * q4 + e] = xe;
            }
        }
        hot_k_pairs<BK>(nat, pairs);
#pragma unroll
        for (int st = 0; st < KSTEPS; ++st)
            qreg[st] = __builtin_bit_cast(h8, (u4){pairs[4 * st], pairs[4 * st + 1], pairs[4 * st + 2], pairs[4 * st + 3]});
        if (OUT) {
            u4 *qn = (u4 *)qn_lds + col * 16 + grp * 4;
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) qn[q4] = (u4){nat[4 * q4], nat[4 * q4 + 1], nat[4 * q4 + 2], nat[4 * q4 + 3]};
        }
    }
    auto qop = [&](int st) { return qreg[st]; };
    // every read of the query slot has returned before the slot is refilled
    wait_lgkm0();
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int s2 = 1; s2 < NS; ++s2) {
        next_unit(qk[s2], qi[s2]);
        issue(qk[s2], qi[s2], ring + s2 * slot_bytes);
    }

    h4 hot_p = {};  // P of the hot tile whose K half was just processed
    int head = 0;  // ring slot of the oldest queue entry
    // Wait for the head slot's loads (the younger slots' loads may stay in flight).
    auto wait_head = [&]() {
        int nwy = 0, nhy = 0;
#pragma unroll
        for (int i = 1; i < NS; ++i) {
            nwy += qk[i] == kWarm;
            nhy += qk[i] == kHotK || qk[i] == kHotV;
        }
        wait_younger<NLW, NLH, NS - 1>(nwy, nhy);
    };
    // Every read of the head slot has landed: refill it with the youngest entry.
    auto advance = [&](unsigned char *slot) {
        wait_lgkm0();
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i + 1 < NS; ++i) {
            qk[i] = qk[i + 1];
            qi[i] = qi[i + 1];
        }
        next_unit(qk[NS - 1], qi[NS - 1]);
        issue(qk[NS - 1], qi[NS - 1], slot);
        head = head + 1 == NS ? 0 : head + 1;
    };
    // Items come from the counter in order, warm units first, so a wave's warm
    // units all precede its hot tiles: two loops over the one ring, so that each
    // loop body updates the accumulators along one path.
    while (qk[0] == kWarm) {
        const int id = qi[0];
        unsigned char *slot = ring + head * slot_bytes;
#ifdef AKV_TIMELINE
        {
            const unsigned long long t0 = AKV_TL_NOW();
            wait_head();
            tl_wait += AKV_TL_NOW() - t0;
            ++tl_items;
        }
#else
        wait_head();
#endif
        if (NG < 4 && id * kUnit + kUnit > nw) {
            // the tail unit: meta rows past the tier's last token may hold bytes from outside it
            const int t = lane & 31;
            if (lane < 32 && t >= nw - id * kUnit) {
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    *(_Float16 *)(slot + L::VS + 2 * (t * NG + g)) = (_Float16)0;
                    *(_Float16 *)(slot + L::VZ + 2 * (t * NG + g)) = (_Float16)0;
                    if (LEG) {
                        *(_Float16 *)(slot + L::KS + 2 * (t * NG + g)) = (_Float16)0;
                        *(_Float16 *)(slot + L::KZ + 2 * (t * NG + g)) = (_Float16)0;
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
        {
            // ---- LDS reads at the top of the unit, issued together (the empty asm with a memory
            //      clobber keeps them above it, so their latencies overlap instead of each read
            //      being waited for before the next is issued): first (block-affine) the lane's
            //      K-meta pair of the prep below, then the lane's packed K rows of both halves
            //      and the V scales of the overflow test.  The prep goes first so that its LDS
            //      write -> read round trip overlaps the K-window work.
            h2 s2v = {}, z2v = {};
            if constexpr (!LEG) {
                s2v = lds_h2(slot + L::KS + 2 * kch_lo, slot + L::KS + 2 * kch_hi);
                z2v = lds_h2(slot + L::KZ + 2 * kch_lo, slot + L::KZ + 2 * kch_hi);
            }
            uint32_t kraw[2][BK];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t *kp = (const uint32_t *)(slot + k_lane + 16 * h * L::KR);
#pragma unroll
                for (int jj = 0; jj < BK; ++jj) kraw[h][jj] = kp[jj];
            }
            h2 vsv = {};
            if (!LEG && lane * 4 < L::VMB) vsv = as_h2(*(const uint32_t *)(slot + L::VS + 4 * lane));
            asm volatile("" ::: "memory");
            // ---- K meta of the block: (s, -2^(10-o) s, z) per channel pair, shared via LDS
            //      and read back per MFMA step; the fast paths hold when no -1024 s overflows
            //      (K and V scales of the unit).  LEG: the lane's 32 channels lie in one group,
            //      so its token has one (s, z) per half, read from the slot; the value is
            //      round16(c s + z) in one fma, rounded once in fp16 (the reference rounds c s + z
            //      in fp32 and then to fp16, so a value may differ by one fp16 ulp at an fp32-rounded
            //      tie: within the attention tolerance), and the symmetric branch
            //      round16((c - half_max) s).
            bool kfast = true;
            h2 ls[2] = {}, lz[2] = {};
            if constexpr (LEG) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int mo = 2 * ((16 * h + col) * NG + (32 * grp) / GV);
                    const _Float16 sv = *(const _Float16 *)(slot + L::KS + mo);
                    const _Float16 zv = symk ? (_Float16)0 : *(const _Float16 *)(slot + L::KZ + mo);
                    ls[h] = (h2){sv, sv};
                    lz[h] = (h2){zv, zv};
                }
            } else {
                const h2 n2 = s2v * (h2){nmul, nmul};
                const uint32_t nb = as_u32(n2);
                kfast = !__builtin_amdgcn_ballot_w64(!finite2(nb));
                uint32_t *kmw = (uint32_t *)kmeta;
                kmw[(0 * 4 + g2) * 16 + pi2] = as_u32(s2v);
                kmw[(1 * 4 + g2) * 16 + pi2] = nb;
                kmw[(2 * 4 + g2) * 16 + pi2] = as_u32(z2v);
                __builtin_amdgcn_wave_barrier();
            }
            KWin<BK> W[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) k_windows<BK>(kraw[h], W[h]);
            // ---- the V fast path holds when no -1024 s of the unit's V scales overflows
            bool vfast;
            {
                bool vfin = true;
                if (!LEG && lane * 4 < L::VMB) {
                    const _Float16 n0 = (_Float16)(-1024.0f);
                    vfin = finite2(as_u32(vsv * (h2){n0, n0}));
                }
                vfast = !__builtin_amdgcn_ballot_w64(!vfin);
            }
            const u4 *kmr = (const u4 *)kmeta;

            const int tok0 = id * kUnit;  // first token of the unit (pair-local warm index)
            // ---- QK of both 16-token halves, step by step (two independent MFMA chains)
            f4 sc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
            if constexpr (LEG) {
#pragma unroll
                for (int st = 0; st < KSTEPS; ++st) {
                    const h8 qst = qop(st);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        h8 a;
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) {
                            const int pi = 4 * st + kk;
                            const uint32_t uu = (k_window_of<BK>(W[h], pi) & km.m[koff<BK>(pi)]) | magic2(koff<BK>(pi));
                            const _Float16 mv = (_Float16)magic_val(koff<BK>(pi)) + hofk;
                            const h2 v = pk_fma(as_h2(uu) - (h2){mv, mv}, ls[h], lz[h]);  // (code - offset) s + z
                            a[2 * kk] = v[0];
                            a[2 * kk + 1] = v[1];
                        }
                        sc[h] = mfma_k32(a, qst, sc[h]);
                    }
                }
            } else if (kfast) {
#pragma unroll
                for (int st = 0; st < KSTEPS; ++st) {
                    const u4 av = kmr[(0 * 4 + grp) * 4 + st], nv = kmr[(1 * 4 + grp) * 4 + st];
                    const u4 zv = kmr[(2 * 4 + grp) * 4 + st];
                    const h8 qst = qop(st);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        h8 a;
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) {
                            const int pi = 4 * st + kk;
                            const uint32_t uu = (k_window_of<BK>(W[h], pi) & km.m[koff<BK>(pi)]) | magic2(koff<BK>(pi));
                            h2 v = pk_fma(as_h2(uu), as_h2(av[kk]), as_h2(nv[kk]));
                            v = v + as_h2(zv[kk]);
                            a[2 * kk] = v[0];
                            a[2 * kk + 1] = v[1];
                        }
                        sc[h] = mfma_k32(a, qst, sc[h]);
                    }
                }
            } else {
#pragma unroll
                for (int st = 0; st < KSTEPS; ++st) {
                    const u4 av = kmr[(0 * 4 + grp) * 4 + st], zv = kmr[(2 * 4 + grp) * 4 + st];
                    const h8 qst = qop(st);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        h8 a;
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) {
                            const int pi = 4 * st + kk;
                            const uint32_t uu = (k_window_of<BK>(W[h], pi) & km.m[koff<BK>(pi)]) | magic2(koff<BK>(pi));
                            const _Float16 mv = (_Float16)magic_val(koff<BK>(pi));
                            const h2 c = as_h2(uu) - (h2){mv, mv};  // the code, exactly
                            h2 v = c * as_h2(av[kk]);
                            v = v + as_h2(zv[kk]);
                            a[2 * kk] = v[0];
                            a[2 * kk + 1] = v[1];
                        }
                        sc[h] = mfma_k32(a, qst, sc[h]);
                    }
                }
            }
            // ---- outlier channels of K: the stored fp16 value replaces the dequantized one,
            //      so q[c] * (value - dequant) joins the dot product.  A channel the
            //      quantizer zeroed has scale = zero = 0 and dequantizes to 0, which skips
            //      the code lookup (taken only when some outlier channel has other meta).
            if constexpr (OUT) {
                const int no = OUT == 1 ? 1 : p.n_out;
                const int *ki = (const int *)(slot + L::KI);  // low words of the int64 indices
                bool lookup = false;
                for (int o = 0; o < no; ++o) {
                    const int c = min(max(ki[2 * o], 0), kD - 1);
                    lookup |= *(const _Float16 *)(slot + L::KS + 2 * c) != (_Float16)0 ||
                              *(const _Float16 *)(slot + L::KZ + 2 * c) != (_Float16)0;
                }
                if (!__builtin_amdgcn_ballot_w64(lookup) && no == 1) {
                    const int c = min(max(ki[0], 0), kD - 1);
                    const float qd = (float)qn_lds[col * kD + c];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const h4 od = *(const h4 *)(slot + L::KO + 2 * (16 * h + 4 * grp));  // tokens 4 grp .. +3
                        // q[c] * value is exact in fp32 (two fp16 factors), so one fma equals the
                        // product-then-add and takes the fp16 operands directly (v_fma_mix)
#pragma unroll
                        for (int i = 0; i < 4; ++i) sc[h][i] = __builtin_fmaf(qd, (float)od[i], sc[h][i]);
                    }
                } else {
                    for (int o = 0; o < no; ++o) {
                        const int c = min(max(ki[2 * o], 0), kD - 1);
                        const _Float16 s_c = *(const _Float16 *)(slot + L::KS + 2 * c);
                        const _Float16 z_c = *(const _Float16 *)(slot + L::KZ + 2 * c);
                        const float qd = (float)qn_lds[col * kD + c];
#pragma unroll
                        for (int h = 0; h < 2; ++h)
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const int t = 16 * h + 4 * grp + i;
                                const float od = (float)*(const _Float16 *)(slot + L::KO + 2 * (t * no + o));
                                const uint32_t code = extract_code(slot + L::KC + t * L::KR, c, BK);
                                const float kd = (float)(_Float16)((_Float16)((_Float16)(float)code * s_c) + z_c);
                                sc[h][i] += qd * (od - kd);
                            }
                    }
                }
            }

            // ---- V: lane (chunk col, tokens 4 grp .. +3 of each half); token pairs per dword
            //      (read here, before the softmax, so the LDS reads are in flight while it runs;
            //      the code reads share one base address and take immediate offsets)
            uint32_t vraw[2][4];
            {
                const lds_cu32 *vq = lds_ptr<uint32_t>(in_vgpr(lds_addr(slot) + (uint32_t)(v_lane & ~3)));
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii) {
                        const int o = (16 * h + ii) * L::VR / 4;
                        if (BV == 3) {  // the chunk's 3 bytes from the aligned 8 around them
                            vraw[h][ii] = __builtin_amdgcn_alignbyte(vq[o + 1], vq[o], v_lane & 3);
                        } else if (BV == 2) {
                            vraw[h][ii] = lds_u16(slot + v_lane + (16 * h + ii) * L::VR);
                        } else {
                            vraw[h][ii] = vq[o];
                        }
                    }
            }
            h2 vs[2][2], vz[2][2];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int pp = 0; pp < 2; ++pp) {
                    const int ta = 16 * h + 2 * pp;  // + 4 grp (in vm_lane)
                    vs[h][pp] = lds_h2(slot + L::VS + vm_lane + ta * NG * 2, slot + L::VS + vm_lane + (ta + 1) * NG * 2);
                    vz[h][pp] = lds_h2(slot + L::VZ + vm_lane + ta * NG * 2, slot + L::VZ + vm_lane + (ta + 1) * NG * 2);
                    if (LEG && symv) vz[h][pp] = (h2){(_Float16)0, (_Float16)0};  // symmetric: no zero-point
                }
            // ---- softmax over the 32 tokens (ragged tail masked; logits stashed)
            if (tok0 + kUnit > nw) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int nvalid = min(4, nw - (tok0 + 16 * h + 4 * grp));
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii)
                        if (ii >= nvalid) sc[h][ii] = -INFINITY;
                }
            }
            if (p.stash) {
                if (st_vec_w && tok0 + kUnit <= nw) {  // a whole unit: two 16-byte stores per lane
                    if (row_valid) {
#pragma unroll
                        for (int h = 0; h < 2; ++h)
                            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, sc[h]), srs, (int)st_w_voff,
                                                                   (tok0 + 16 * h) * 4, 16);
                    }
                } else {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int t0 = tok0 + 16 * h;
                        stash4(p, strow, row_valid, warm_base + t0 + 4 * grp, sc[h], min(4, nw - (t0 + 4 * grp)),
                               st_vec_w, srs, sbase);
                    }
                }
            }
            const h8 pop = softmax32(stt, sc[0], sc[1], sl2);

            uint32_t win[2][2][VSlot<BV>::NW];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int pp = 0; pp < 2; ++pp) v_windows<BV>(vraw[h][2 * pp], vraw[h][2 * pp + 1], win[h][pp]);
            // one outlier channel per block (the common case): its stored value replaces the
            // dequantized one inside the PV operand (lanes of its chunk, MFMA kk1), so only
            // its zero term needs a correction afterwards
            int kk1 = -1;
            bool gsel1 = false;
            uint32_t ov1[4] = {0u, 0u, 0u, 0u};
            if constexpr (OUT) {
                if (OUT == 1 || p.n_out == 1) {
                    const int c = __builtin_amdgcn_readfirstlane(min(max(*(const int *)(slot + L::VI), 0), kD - 1));
                    kk1 = c & 7;
                    gsel1 = col == (c >> 3);
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        ov1[q] = *(const uint32_t *)(slot + L::VO + 2 * (16 * (q >> 1) + 4 * grp + 2 * (q & 1)));
                }
            }
            // One MFMA per channel chunk for both paths: the fast operand is always formed and a
            // block whose -2^(10-o) s overflows (rare) overwrites it with the exact two-op form.
            // A second MFMA on the accumulator in another branch would make the compiler keep
            // the accumulators in two register sets and copy them every unit.
            {
                h2 vn[2][2][v_noffs<BV>()];
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int pp = 0; pp < 2; ++pp)
#pragma unroll
                        for (int oi = 0; oi < v_noffs<BV>(); ++oi) {
                            const _Float16 m = (_Float16)(-magic_val(oi * v_ostep<BV>()));
                            vn[h][pp][oi] = vs[h][pp] * (h2){m, m};
                        }
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    uint32_t d[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int h = q >> 1, pp = q & 1;
                        const uint32_t uu = (win[h][pp][vwin<BV>(kk)] & vmk.m[voff<BV>(kk)]) | magic2(voff<BV>(kk));
                        if constexpr (LEG) {  // round16((code - offset) s + z), z of the token pair
                            const _Float16 mv = (_Float16)magic_val(voff<BV>(kk)) + hofv;
                            d[q] = as_u32(pk_fma(as_h2(uu) - (h2){mv, mv}, vs[h][pp], vz[h][pp]));
                        } else {
                            d[q] = as_u32(pk_fma(as_h2(uu), vs[h][pp], vn[h][pp][voff<BV>(kk) / v_ostep<BV>()]));
                        }
                    }
                    if (!LEG && __builtin_expect(!vfast, 0)) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const int h = q >> 1, pp = q & 1;
                            const uint32_t uu = (win[h][pp][vwin<BV>(kk)] & vmk.m[voff<BV>(kk)]) | magic2(voff<BV>(kk));
                            const _Float16 mv = (_Float16)magic_val(voff<BV>(kk));
                            const h2 c = as_h2(uu) - (h2){mv, mv};
                            d[q] = as_u32(c * vs[h][pp]);
                        }
                    }
                    if (OUT && kk == kk1) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) d[q] = gsel1 ? ov1[q] : d[q];
                    }
                    stt.acc[kk] = mfma_k32(__builtin_bit_cast(h8, (u4){d[0], d[1], d[2], d[3]}), pop, stt.acc[kk]);
                }
            }
            if constexpr (!LEG) {  // the zero-points of the block-affine V: sum_t P z per group
                const h8 az8 = __builtin_bit_cast(h8, (u4){as_u32(vz[0][0]), as_u32(vz[0][1]), as_u32(vz[1][0]), as_u32(vz[1][1])});
                stt.accz = mfma_k32(az8, pop, stt.accz);
            }
            // ---- outlier channels of V: channel c of chunk c/8 took round16(code s) + z
            //      (z through accz).  With one outlier channel its value already replaced
            //      round16(code s) in the PV operand and one MFMA removes the z term; with more,
            //      three exact MFMAs per channel add sum_t P (value - round16(code s) - z) to its
            //      accumulator, in the lanes of that chunk only
            if constexpr (OUT) {
                const int no = OUT == 1 ? 1 : p.n_out;
                const int *vi = (const int *)(slot + L::VI);
                if (no == 1) {  // the value went in above; take out the zero term accz added
                    uint32_t az[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) az[q] = gsel1 ? (as_u32(vz[q >> 1][q & 1]) ^ 0x80008000u) : 0u;
                    const h8 a3 = __builtin_bit_cast(h8, (u4){az[0], az[1], az[2], az[3]});
                    switch (kk1) {
                        case 0: stt.acc[0] = mfma_k32(a3, pop, stt.acc[0]); break;
                        case 1: stt.acc[1] = mfma_k32(a3, pop, stt.acc[1]); break;
                        case 2: stt.acc[2] = mfma_k32(a3, pop, stt.acc[2]); break;
                        case 3: stt.acc[3] = mfma_k32(a3, pop, stt.acc[3]); break;
                        case 4: stt.acc[4] = mfma_k32(a3, pop, stt.acc[4]); break;
                        case 5: stt.acc[5] = mfma_k32(a3, pop, stt.acc[5]); break;
                        case 6: stt.acc[6] = mfma_k32(a3, pop, stt.acc[6]); break;
                        default: stt.acc[7] = mfma_k32(a3, pop, stt.acc[7]); break;
                    }
                }
                for (int o = 0; o < no && no > 1; ++o) {
                    const int c = min(max(vi[2 * o], 0), kD - 1);
                    const bool gsel = col == (c >> 3);
                    uint32_t av[4], az[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int h = q >> 1, pp = q & 1, t = 16 * h + 4 * grp + 2 * pp;
                        const uint32_t ov = no == 1 ? *(const uint32_t *)(slot + L::VO + 2 * t)
                                                    : as_u32(lds_h2(slot + L::VO + 2 * (t * no + o),
                                                                    slot + L::VO + 2 * ((t + 1) * no + o)));
                        av[q] = gsel ? ov : 0u;
                        az[q] = gsel ? (as_u32(vz[h][pp]) ^ 0x80008000u) : 0u;
                    }
                    // the code of channel c for the lane's token pairs, selected at run time
                    // (offset and window are uniform), then round16(code s) exactly
                    const int kk = c & 7, off = voff<BV>(kk), wsel = vwin<BV>(kk);
                    const uint32_t msk = (((1u << BV) - 1u) << off) * 0x00010001u;
                    const _Float16 mv = (_Float16)magic_val(off);
                    uint32_t ad[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int h = q >> 1, pp = q & 1;
                        uint32_t wv = win[h][pp][0];
#pragma unroll
                        for (int wi = 1; wi < VSlot<BV>::NW; ++wi) wv = wsel == wi ? win[h][pp][wi] : wv;
                        const uint32_t uu = (wv & msk) | magic2(off);
                        const h2 d = (as_h2(uu) - (h2){mv, mv}) * vs[h][pp];
                        ad[q] = gsel ? (as_u32(d) ^ 0x80008000u) : 0u;
                    }
                    const h8 a1 = __builtin_bit_cast(h8, (u4){av[0], av[1], av[2], av[3]});
                    const h8 a2 = __builtin_bit_cast(h8, (u4){ad[0], ad[1], ad[2], ad[3]});
                    const h8 a3 = __builtin_bit_cast(h8, (u4){az[0], az[1], az[2], az[3]});
                    auto fix = [&](f4 &acc) {
                        acc = mfma_k32(a1, pop, acc);
                        acc = mfma_k32(a2, pop, acc);
                        acc = mfma_k32(a3, pop, acc);
                    };
                    switch (kk) {
                        case 0: fix(stt.acc[0]); break;
                        case 1: fix(stt.acc[1]); break;
                        case 2: fix(stt.acc[2]); break;
                        case 3: fix(stt.acc[3]); break;
                        case 4: fix(stt.acc[4]); break;
                        case 5: fix(stt.acc[5]); break;
                        case 6: fix(stt.acc[6]); break;
                        default: fix(stt.acc[7]); break;
                    }
                }
            }
        }
        advance(slot);
    }
    AKV_TL(2, AKV_TL_NOW());
    while (qk[0] != kNone) {
        const int k = qk[0];
        const int id = qi[0];
        unsigned char *slot = ring + head * slot_bytes;
#ifdef AKV_TIMELINE
        {
            const unsigned long long t0 = AKV_TL_NOW();
            wait_head();
            tl_wait += AKV_TL_NOW() - t0;
            ++tl_items;
        }
#else
        wait_head();
#endif
        if (k == kHotK) {
            // ---- hot K tile: 16 tokens x 256 B; lane = (token col, 32 channels of group grp)
            uint32_t nat[16], pairs[16];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const u4 x = *(const u4 *)(slot + col * 256 + grp * 64 + 16 * q4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t xe = x[e];
                    nat[4 * q4 + e] = xe;
                }
            }
            hot_k_pairs<BK>(nat, pairs);
            f4 sh = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < KSTEPS; ++st)
                sh = mfma_k32(__builtin_bit_cast(h8, (u4){pairs[4 * st], pairs[4 * st + 1], pairs[4 * st + 2], pairs[4 * st + 3]}),
                              qop(st), sh);
            const int t0 = id * 16;
            const int nvalid = min(4, nh - (t0 + 4 * grp));
            if (t0 + 16 > nh) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii)
                    if (ii >= nvalid) sh[ii] = -INFINITY;
            }
            stash4(p, strow, row_valid, hot_base + t0 + 4 * grp, sh, nvalid, st_vec_h, srs, sbase);
            hot_p = softmax16(stt, sh, sl2);
        } else {
            // ---- hot V tile: lane = (chunk col, tokens 4 grp .. +3)
            u4 w[4];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) w[ii] = *(const u4 *)(slot + (4 * grp + ii) * 256 + col * 16);
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const uint32_t sel = (kk & 1) ? 0x07060302u : 0x05040100u;
                const uint32_t lo = perm(w[1][kk / 2], w[0][kk / 2], sel);
                const uint32_t hi = perm(w[3][kk / 2], w[2][kk / 2], sel);
                stt.acc[kk] = mfma_k16(__builtin_bit_cast(h4, (u2){lo, hi}), hot_p, stt.acc[kk]);
            }
        }
        advance(slot);
    }

    // ---- merge the waves (the ring memory is reused): every wave rescales its
    //      rows to the workgroup maximum, then the 12 states are summed
#ifdef AKV_TIMELINE
    AKV_TL(3, AKV_TL_NOW());
    AKV_TL(7, tl_items);
    AKV_TL(8, tl_wait);
    {
        unsigned xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        AKV_TL(9, xcc & 7u);
    }
#endif
    wait_vm<0>();
    stt.l = wsum16(stt.l);
    __syncthreads();
    float *mlds = (float *)smem;                   // [W][16] running maxima
    float *llds = mlds + NW * 16;              // [W][16] rescaled sums
    float *alds = llds + NW * 16;              // [W][16][kAccRow] rescaled accumulators
    if (grp == 0) mlds[wave * 16 + col] = stt.m2;
    __syncthreads();
    {
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) mx = fmaxf(mx, mlds[w * 16 + col]);
        const float fw = (stt.m2 == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(stt.m2 - mx);
        if (grp == 0) llds[wave * 16 + col] = stt.l * fw;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
                alds[(wave * 16 + col) * kAccRow + 8 * (4 * grp + ii) + kk] = (stt.acc[kk][ii] + stt.accz[ii]) * fw;
    }
    __syncthreads();
    const int64_t bhc = bh * p.nchunk + chunk;
    constexpr int PS = kD + 4;  // partial row: (m, l, pad, pad, acc[D])
    const int64_t pstride = (int64_t)p.prows * PS;
    float *part = p.part + (bhc * p.nsplit + split) * pstride;
    const bool fused = p.split_ctr != nullptr;
    // this (batch, kv-head, row chunk)'s partials as a buffer; the fused merge
    // moves them with write-through stores and coherent loads (cache policy sc1)
    const __amdgpu_buffer_rsrc_t prs = make_rsrc(p.part + bhc * p.nsplit * pstride, (uint32_t)(p.nsplit * pstride * 4));
    constexpr int kSc1 = 16;  // cache-policy bit sc1: coherent at device scope
    const int tid = threadIdx.x;
    AKV_TL(11, AKV_TL_NOW());
    if (tid < nrows * (kD / 4)) {  // thread = (row, channel quad); 512 <= 64 * NW
        const int rr = tid / (kD / 4), c4 = tid % (kD / 4);
        f4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < NW; ++w) a += *(const f4 *)(alds + (w * 16 + rr) * kAccRow + 4 * c4);
        const int off = (int)((split * pstride + rr * PS) * 4);
        if (fused) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, a), prs, off + 16 + 16 * c4, 0, kSc1);
        else *(f4 *)(part + rr * PS + 4 + 4 * c4) = a;
        if (c4 == 0) {
            float mx = -INFINITY, l = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                mx = fmaxf(mx, mlds[w * 16 + rr]);
                l += llds[w * 16 + rr];
            }
            if (fused) __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, (f2){mx, l}), prs, off, 0, kSc1);
            else {
                part[rr * PS + 0] = mx;
                part[rr * PS + 1] = l;
            }
        }
    }
    if (!fused) {
        AKV_TL_FLUSH();
        return;
    }

    // ---- split merge in the kernel: the workgroup whose partial completes the
    //      (batch, kv-head, row chunk) merges all of them.  The partials were
    //      written through to the device coherence point (and the writer's L2);
    //      waiting for the stores before the counter increment orders them before
    //      it.  The merge reads them from its own L2 when every partial came from
    //      its XCD, else from the coherence point.  The counter returns to zero.
    wait_vm<0>();
    AKV_TL(4, AKV_TL_NOW());
    __syncthreads();
    if (tid == 0) {
        // one byte per XCD counts the partials written from it
        unsigned xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
        xcc &= 7u;
        const uint64_t inc = 1ull << (8 * xcc);
        const uint64_t now = __hip_atomic_fetch_add(p.split_ctr + bhc, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + inc;
        unsigned total = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) total += (unsigned)(now >> (8 * i)) & 255u;
        // 0: not last; 1: last; 2: last, and every partial came from this XCD (its L2 holds them)
        *work = total != (unsigned)p.nsplit ? 0u : (((unsigned)(now >> (8 * xcc)) & 255u) == (unsigned)p.nsplit ? 2u : 1u);
    }
    __syncthreads();
    const unsigned role = *work;
    AKV_TL(5, AKV_TL_NOW() * 4ull + role);
    if (role == 0u) {
        AKV_TL_FLUSH();
        return;
    }
    // The count returns to zero from the workgroup's last thread when that thread merges
    // nothing (a merging wave would wait for this store with its loads: vmcnt counts stores
    // and loads in issue order).
    if (tid == (nrows * (kD / 4) < 64 * NW ? 64 * NW - 1 : 0))
        __hip_atomic_store(p.split_ctr + bhc, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid >= nrows * (kD / 4)) {
        AKV_TL_FLUSH();
        return;
    }
    {
        const int rr = tid / (kD / 4), c4 = tid % (kD / 4);
        float M = -INFINITY, L = 0.f;
        f4 a = {0.f, 0.f, 0.f, 0.f};
        if (role == 2u) merge_partials<1>(prs, p.nsplit, pstride, rr, c4, M, L, a);    // L2-coherent loads
        else merge_partials<kSc1>(prs, p.nsplit, pstride, rr, c4, M, L, a);            // device-coherent loads
        if (tid == 0) AKV_TL(12, AKV_TL_NOW());
        const int r = row0 + rr;
        const int rq2 = (int)fast_div((uint32_t)r, p.fd_m);
        const int h = kvh * p.g + rq2, m = r - rq2 * p.M;
        const int64_t row = (int64_t)(b * p.Hq + h) * p.M + m;
        const h4 ov = {(_Float16)(a[0] / L), (_Float16)(a[1] / L), (_Float16)(a[2] / L), (_Float16)(a[3] / L)};
        *(h4 *)(p.out + row * kD + 4 * c4) = ov;
        if (tid == 0) AKV_TL(6, AKV_TL_NOW());
        if (c4 == 0 && p.rowstats) {
            p.rowstats[2 * row] = M;
            p.rowstats[2 * row + 1] = 1.0f / (L * (1.0f / 128.0f));  // 1 / L, the 2^7 probability scale undone
        }
    }
    AKV_TL_FLUSH();
}

// LDS slot of the fast kernel: one warm unit, or one 16-token hot K or V half.
// K meta of a unit: two 256-byte block rows (block-affine) or two 64 NG-byte token
// rows of groups (legacy).
int64_t decode_fast_slot_bytes(int kb, int vb, int Gv, int n_out, bool legacy) {
    const int NG = kD / Gv;
    int64_t warm = (int64_t)kUnit * 16 * (kb + vb) + (legacy ? 128 * NG : 512) + 128 * NG +
                   (n_out > 0 ? kOutBytes : 0);
    int64_t s = warm > 4096 ? warm : 4096;
    return (s + 255) / 256 * 256;
}
// LDS of one workgroup: W waves x (NS slots + K meta scratch) + the item
// counter; the end-of-split merge reuses the rings (slots are >= 4 KiB, so the
// merge never reaches the item counter, which also carries the last-arrival flag).
static_assert(kWaves * (kNS * 4096 + kKmetaBytes) >= (2 * kWaves * 16 + kWaves * 16 * kAccRow) * 4,
              "merge area overlaps the item counter");
static_assert(kWavesOut * (kNSOut * 4096 + kKmetaBytes) >= (2 * kWavesOut * 16 + kWavesOut * 16 * kAccRow) * 4,
              "merge area overlaps the item counter");
int64_t decode_fast_lds_bytes(int64_t slot, int n_out) {
    const int nw = n_out > 1 ? kWavesOut : kWaves, ns = n_out > 1 ? kNSOut : kNS;
    // the item counter, plus the natural-order query rows for the outlier corrections
    const int64_t ring = nw * (ns * slot + kKmetaBytes) + 16 + (n_out > 0 ? kQldsBytes : 0);
    const int64_t merge = (int64_t)(2 * nw * 16 + nw * 16 * kAccRow) * 4;
    return ring > merge ? ring : merge;
}
int decode_fast_waves(int n_out) { return n_out > 1 ? kWavesOut : kWaves; }

bool decode_fast_legacy_shape(int D, int bits, int group_size, int meta_dtype) {
    return D == kD && (bits == 2 || bits == 4) && (group_size == 32 || group_size == 64 || group_size == 128) &&
           meta_dtype == AKV_DT_F16;
}

bool decode_fast_meta_aligned(int64_t rows_per_head, int Gv, int64_t heads) {
    const int ng = kD / Gv;
    return ng == 4 || heads <= 1 || (rows_per_head * ng * 2) % 16 == 0;
}

bool decode_fast_eligible(const DecodeParams &p, int wk) {
    if (wk == AKV_WARM_LEGACY) {
        if (!(decode_fast_legacy_shape(p.D, p.kc_row * 8 / kD, p.gs, p.meta_dt) && p.kc_row == p.vc_row &&
              p.Gv == p.gs && decode_fast_meta_aligned(p.w_stride, p.gs, p.warm_heads)))
            return false;
        return p.slot_bytes > 0 && decode_fast_lds_bytes(p.slot_bytes, 0) <= kLdsCap;
    }
    if (!(wk == AKV_WARM_AFFINE && p.D == kD && p.T % kUnit == 0 && (p.Gv == 32 || p.Gv == 64 || p.Gv == 128) &&
          decode_fast_meta_aligned(p.n_warm, p.Gv, (int64_t)p.B * p.Hkv)))
        return false;
    // outlier channels: up to kMaxOut per block, V groups of 32 channels; the ring must fit the LDS
    if (p.n_out != 0 && !(p.n_out <= kMaxOut && p.Gv == 32 && p.k_odata && p.v_odata && p.k_oidx && p.v_oidx))
        return false;
    return p.slot_bytes > 0 && decode_fast_lds_bytes(p.slot_bytes, p.n_out) <= kLdsCap;
}

template <int BK, int BV, int NG, int NS, int OUT, bool LEG>
static hipError_t launch_fast_ns(const DecodeParams &p, hipStream_t s) {
    const dim3 grid((unsigned)(p.nsplit * p.Hkv * p.B * p.nchunk));  // decoded in the kernel
    const size_t lds = (size_t)decode_fast_lds_bytes(p.slot_bytes, OUT ? p.n_out : 0);
    // raise the dynamic LDS cap above 64 KiB once per device (a bit per device index;
    // host threads that race here both set it, which is harmless)
    static std::atomic<uint64_t> attr_devs{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = (dev >= 0 && dev < 64) ? 1ull << dev : 0ull;
    if (!bit || !(attr_devs.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void *)decode_fast_kernel<BK, BV, NG, NS, OUT, LEG>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, kLdsCap);
        if (e != hipSuccess) return e;
        attr_devs.fetch_or(bit, std::memory_order_release);
    }
    hipLaunchKernelGGL((decode_fast_kernel<BK, BV, NG, NS, OUT, LEG>), grid, dim3(64 * FastCfg<OUT>::NW), lds, s, p);
    return hipGetLastError();
}

template <int BK, int BV, int NG, bool LEG>
static hipError_t launch_fast(const DecodeParams &p, hipStream_t s) {
    return launch_fast_ns<BK, BV, NG, kNS, 0, LEG>(p, s);
}

template <int BK, int BV, bool LEG>
static hipError_t launch_fast_ng(const DecodeParams &p, hipStream_t s) {
    if (!LEG && p.n_out > 0)
        return p.Gv != 32 ? hipErrorInvalidValue
               : p.n_out == 1 ? launch_fast_ns<BK, BV, 4, kNS, 1, false>(p, s)
                              : launch_fast_ns<BK, BV, 4, kNSOut, kMaxOut, false>(p, s);
    if (p.Gv == 32) return launch_fast<BK, BV, 4, LEG>(p, s);
    if (p.Gv == 64) return launch_fast<BK, BV, 2, LEG>(p, s);
    if (p.Gv == 128) return launch_fast<BK, BV, 1, LEG>(p, s);
    return hipErrorInvalidValue;
}

// Timeline of the last launches (timeline build only): copy / clear the per-wave words.
int64_t decode_fast_timeline_words() {
#ifdef AKV_TIMELINE
    return kTlCap;
#else
    return 0;
#endif
}
hipError_t decode_fast_timeline_fetch(unsigned long long *host, int64_t words) {
#ifdef AKV_TIMELINE
    if (words > kTlCap) words = kTlCap;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_akv_timeline), (size_t)words * 8, 0, hipMemcpyDeviceToHost);
#else
    (void)host;
    (void)words;
    return hipErrorNotSupported;
#endif
}
hipError_t decode_fast_timeline_clear(hipStream_t s) {
#ifdef AKV_TIMELINE
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_akv_timeline));
    if (e != hipSuccess) return e;
    return hipMemsetAsync(ptr, 0, sizeof(unsigned long long) * kTlCap, s);
#else
    (void)s;
    return hipErrorNotSupported;
#endif
}

hipError_t decode_fast_split_launch(const DecodeParams &p, int kb, int vb, int wk, hipStream_t s) {
    if (wk == AKV_WARM_LEGACY) {
        if (kb == 2 && vb == 2) return launch_fast_ng<2, 2, true>(p, s);
        if (kb == 4 && vb == 4) return launch_fast_ng<4, 4, true>(p, s);
        return hipErrorInvalidValue;
    }
#define AKV_FKV(a, b) \
    if (kb == a && vb == b) return launch_fast_ng<a, b, false>(p, s);
    AKV_FKV(2, 2) AKV_FKV(2, 3) AKV_FKV(2, 4) AKV_FKV(3, 2) AKV_FKV(3, 3) AKV_FKV(3, 4) AKV_FKV(4, 2) AKV_FKV(4, 3)
    AKV_FKV(4, 4)
#undef AKV_FKV
    return hipErrorInvalidValue;
}

}  // namespace akv
